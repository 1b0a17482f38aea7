"""GPU parity of mask-table rows built on the device from a byte-level DFA
(tgs_mask_rows_from_dfa) against the DFA replay oracle, read back two
ways: the table's words straight from the device (tgs_mask_table_get), and
through the sampler itself (a greedy row over zero logits with mask_state =
the built row reports 0 for allowed ids and -inf for the rest in
post_logits).  Bit-exact."""
import numpy as np
import pytest

import gpu_harness as H

pytestmark = pytest.mark.gpu


def _vocab(g, V):
    pieces = [b"[", b"]", b"POINT", b":", b"none", b",", b"CLICK", b"TYPE", b"SCROLL", b"up", b"down", b"KEY",
              b"+", b"OPEN_APP", b" ", b"_", b"-", b"\n", b"\xc3\xa9", b"\xe2\x80", b"hello", b"12", b"9", b"x", b"A"]
    toks = [b""]
    for _ in range(V - 2):
        if g.random() < 0.6:
            toks.append(b"".join(g.choice(pieces) for _ in range(g.integers(1, 4))))
        else:
            toks.append(bytes(g.integers(32, 127, size=g.integers(1, 24)).astype(np.uint8)))
    toks.append(bytes(range(65, 65 + 40)))  # longer than the bytes read up front
    return toks


def test_tool_tag_rows_built_on_device(sampler, oracle):
    import torch

    import tinygpt_amd as tg
    from tinygpt_amd import grammar as G

    g = np.random.default_rng(21)
    V = 40000
    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    toks = _vocab(g, V)
    off, data = G.token_csr(toks)
    hist = [b"", b"ok ", b"ok [", b"ok [POINT:", b"ok [POINT:1", b"ok [POINT:12,3:Sa", b"[TYPE:abc",
            b"[SCROLL:up:", b"[KEY:cmd", b"[OPEN_APP:Sa 1", b"[POINT:none]"]
    states = np.array([d.walk(0, h) for h in hist], np.int32)
    assert (states >= 0).all() and d.complete[states[-1]]
    n = len(states)
    sampler.set_mask_table(np.full((2 * n + 1, (V + 31) // 32), 0xFFFFFFFF, np.uint32), V)
    dev = "cuda:0"
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    rows = np.arange(n, dtype=np.int32)
    H.log(f"case mask build: V={V} dfa={d.n} states={n}")
    bc, ct = d.byte_classes()
    comp = T(d.complete.astype(np.uint8))
    # the 40-class table (in LDS) fills rows [0, n), the full 256-column
    # table (read from global memory) rows [n, 2n): both against one oracle
    sampler.mask_rows_from_dfa(T(bc), T(ct), comp, T(off), T(data), T(states), T(rows), eos=7)
    sampler.mask_rows_from_dfa(T(np.arange(256, dtype=np.uint8)), T(d.trans), comp, T(off), T(data), T(states),
                               T(rows + n), eos=7)
    # rows outside the table are skipped
    sampler.mask_rows_from_dfa(T(bc), T(ct), comp, T(off), T(data), T(states[:2]),
                               T(np.array([-1, 2 * n + 1], np.int32)))
    torch.cuda.synchronize()
    want = oracle.dfa_mask_rows(d.trans, d.complete, toks, states, eos=7)
    R = 2 * n + 1
    params = tg.make_params(R, temperature=0.0, mask_state=list(range(R)))
    post = torch.full((R, V), float("nan"), dtype=torch.float32, device=dev)
    sampler.sample(torch.zeros(R, V, dtype=torch.float32, device=dev), tg.params_to_device(params, dev),
                   torch.zeros(R, dtype=torch.float32, device=dev), vocab=V, debug={"post_logits": post})
    torch.cuda.synchronize()
    got = post.cpu().numpy()
    direct = H.table_bits(sampler, np.arange(R), V)  # the table's words themselves
    for i in range(2 * n):
        allowed = np.array([(int(want[i % n, v >> 5]) >> (v & 31)) & 1 for v in range(V)], dtype=bool)
        np.testing.assert_array_equal(got[i] == 0.0, allowed, err_msg=f"row {i} ({hist[i % n]!r})")
        np.testing.assert_array_equal(direct[i], allowed, err_msg=f"table row {i} ({hist[i % n]!r})")
        assert np.all(np.isneginf(got[i][~allowed]))
    assert direct[2 * n].all()
    assert (got[2 * n] == 0.0).all()  # the untouched last row still allows everything
    H.log("case mask build: ok")



def test_every_tool_tag_state_both_tables(sampler, oracle):
    """Rows for all states of the tool-tag DFA (many workgroup rows of both
    kernels) through the class table in LDS and the 256-column table read
    from global memory, bit-exact against the DFA replay oracle."""
    import torch

    from tinygpt_amd import grammar as G

    g = np.random.default_rng(22)
    V = 6000
    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    toks = _vocab(g, V)
    off, data = G.token_csr(toks)
    n = d.n
    states = np.arange(n, dtype=np.int32)
    want = oracle.dfa_mask_rows(d.trans, d.complete, toks, states, eos=7)
    bits = np.packbits(np.unpackbits(want.view(np.uint8), axis=1, bitorder="little")[:, :V], axis=1,
                       bitorder="little")
    dev = "cuda:0"
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    bc, ct = d.byte_classes()
    comp = T(d.complete.astype(np.uint8))
    for name, byte_class, trans in (("lds", bc, ct), ("global", np.arange(256, dtype=np.uint8), d.trans)):
        H.log(f"case mask build all states: {name} table, {n} states, V={V}")
        sampler.set_mask_table(np.zeros((n, (V + 31) // 32), np.uint32), V)
        sampler.mask_rows_from_dfa(T(byte_class), T(trans), comp, T(off), T(data), T(states), T(states), eos=7)
        for r0 in range(0, n, 512):
            rows = list(range(r0, min(n, r0 + 512)))
            np.testing.assert_array_equal(_read_rows(sampler, rows, V), bits[r0:r0 + len(rows)],
                                          err_msg=f"{name} rows {r0}..")

@pytest.mark.gpu
def test_mask_build_rejects_bad_arguments(sampler):
    """Argument errors are reported on the host, before any launch."""
    import ctypes as C

    import torch

    from tinygpt_amd import grammar as G

    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    bc, ct = d.byte_classes()
    toks = [b"", b"[", b"ab"]
    off, data = G.token_csr(toks)
    dev = "cuda:0"
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    dbc, dct, dcomp = T(bc), T(ct), T(d.complete.astype(np.uint8))
    doff, ddata, dst, drow = T(off), T(data), T(np.zeros(1, np.int32)), T(np.zeros(1, np.int32))
    sampler.set_mask_table(np.full((2, 1), 0xFFFFFFFF, np.uint32), len(toks))
    L, h = sampler._L, sampler._h
    p = lambda t: C.c_void_p(t.data_ptr())
    ncls = ct.shape[1]

    def call(byte_class=dbc, n_cls=ncls, n_dfa=d.n, n_tokens=len(toks), eos=-1, n=1, n_bytes=ddata.numel()):
        return L.tgs_mask_rows_from_dfa(h, byte_class if byte_class is None else p(byte_class), p(dct), n_cls,
                                        p(dcomp), n_dfa, p(doff), p(ddata), n_bytes, n_tokens, eos, p(dst), p(drow),
                                        n, None)

    assert call() == 0
    assert call(n_cls=0) == -1
    assert call(n_cls=257) == -1
    assert call(n_dfa=0) == -1
    assert call(eos=len(toks)) == -1
    assert call(eos=-2) == -1
    assert call(n=-1) == -1
    assert call(byte_class=None) == -1
    assert call(n_bytes=-1) == -1
    assert call(n_tokens=100) != 0  # more tokens than the table's vocabulary
    assert call(n=0) == 0
    torch.cuda.synchronize()


def _read_rows(sampler, rows, V):
    import torch

    import tinygpt_amd as tg

    dev = "cuda:0"
    params = tg.make_params(len(rows), temperature=0.0, mask_state=list(rows))
    post = torch.empty(len(rows), V, dtype=torch.float32, device=dev)
    sampler.sample(torch.zeros(len(rows), V, device=dev), tg.params_to_device(params, dev),
                   torch.zeros(len(rows), device=dev), vocab=V, debug={"post_logits": post})
    torch.cuda.synchronize()
    bits = (post == 0).cpu().numpy()
    np.testing.assert_array_equal(bits, H.table_bits(sampler, rows, V), err_msg="table words differ from the sampler's view")
    return np.packbits(bits, axis=1, bitorder="little").view(np.uint8)


def test_mask_table_update_batches(sampler):
    """tgs_mask_table_update: a consecutive run (one copy), scattered states
    with a repeat (one upload, one scatter launch: the last repeat wins),
    rows left alone keep their bits, and a bad state changes nothing."""
    V, n = 1000, 64
    words = (V + 31) // 32
    g = np.random.default_rng(77)
    table = g.integers(0, 2**32, size=(n, words), dtype=np.uint64).astype(np.uint32)
    table[:, -1] &= np.uint32((1 << (V % 32)) - 1)
    sampler.set_mask_table(table, V)
    expect = table.copy()

    def check(what):
        got = _read_rows(sampler, range(n), V)
        want = np.unpackbits(expect.view(np.uint8), axis=1, bitorder="little")[:, :V]
        want = np.packbits(want, axis=1, bitorder="little")
        np.testing.assert_array_equal(got, want, err_msg=what)

    new = g.integers(0, 2**32, size=(5, words), dtype=np.uint64).astype(np.uint32)
    new[:, -1] &= np.uint32((1 << (V % 32)) - 1)
    H.log("mask update: consecutive run 10..14")
    sampler.update_mask_rows(np.arange(10, 15), new)
    expect[10:15] = new
    check("consecutive run")
    states = np.array([3, 40, 7, 40, 63], np.int32)
    new = g.integers(0, 2**32, size=(5, words), dtype=np.uint64).astype(np.uint32)
    new[:, -1] &= np.uint32((1 << (V % 32)) - 1)
    H.log("mask update: scattered states with a repeat")
    sampler.update_mask_rows(states, new)
    for i, s in enumerate(states):
        expect[s] = new[i]
    check("scattered")
    H.log("mask update: a state out of range")
    with pytest.raises(Exception):
        sampler.update_mask_rows(np.array([1, n], np.int32), new[:2])
    check("rejected update")


def test_byte_level_token_table_rows(sampler, oracle):
    """Rows over the byte-level model's token table as the server builds it
    (token_bytes_table: ids 128-255 decode to U+FFFD), for every tool-tag
    DFA state, built on the device and read back through the sampler,
    bit-exact against the DFA replay oracle; no row allows ids 128-255,
    whose table bytes EF BF BD the tool-tag language never holds."""
    import torch

    import tinygpt_amd as tg
    from tinygpt_amd import grammar as G

    V = 256
    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    toks = G.token_bytes_table(V)
    off, data = G.token_csr(toks)
    states = np.arange(d.n, dtype=np.int32)
    n = len(states)
    sampler.set_mask_table(np.full((n, (V + 31) // 32), 0xFFFFFFFF, np.uint32), V)
    dev = "cuda:0"
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    H.log(f"case byte-level token table: V={V} states={n}")
    bc, ct = d.byte_classes()
    sampler.mask_rows_from_dfa(T(bc), T(ct), T(d.complete.astype(np.uint8)), T(off), T(data), T(states),
                               T(np.arange(n, dtype=np.int32)))
    params = tg.make_params(n, temperature=0.0, mask_state=list(range(n)))
    post = torch.full((n, V), float("nan"), dtype=torch.float32, device=dev)
    # the batch's hint (every row greedy) keeps these V = 256 rows on the k64
    # kernel, the path the byte-level decode loop runs
    sampler.sample(torch.zeros(n, V, dtype=torch.float32, device=dev), tg.params_to_device(params, dev),
                   torch.zeros(n, dtype=torch.float32, device=dev), vocab=V, debug={"post_logits": post},
                   hint=tg.batch_hint(params, V))
    torch.cuda.synchronize()
    got = post.cpu().numpy() == 0.0
    want = oracle.dfa_mask_rows(d.trans, d.complete, toks, states, eos=-1)
    bits = ((want[:, np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1).astype(bool)
    np.testing.assert_array_equal(got, bits)
    assert not got[:, 128:].any()
    H.log("case byte-level token table: ok")
