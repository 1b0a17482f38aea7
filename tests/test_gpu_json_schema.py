"""JSON-schema grammar rows on the device (GPU): rows built by
JsonSchemaConstraint through tgs_mask_rows_from_dfa against the oracle's
clone-and-replay masker (oracle/json_fsm.py, LogitsMasker.mask,
ConstrainedGen.swift:805-822), the reference's masker known-answer tests
(ConstrainedGenTests.swift:228-270) on the device, and a constrained
decoding loop whose every sampled token the oracle allows."""
import json

import numpy as np
import pytest

import json_fsm as O
import json_schema_util as U
from gpu_harness import log, table_bits

pytestmark = pytest.mark.gpu


def read_rows(sampler, rows, V):
    """Allowed ids of mask-table rows, read back through greedy rows over
    zero logits (post-mask logits: 0 allowed, -inf not), and checked equal
    to the table's words read straight from the device."""
    import torch

    import tinygpt_amd as tg

    dev = "cuda:0"
    B = len(rows)
    params = tg.make_params(B, temperature=0.0, mask_state=[int(r) for r in rows])
    post = torch.empty(B, V, dtype=torch.float32, device=dev)
    sampler.sample(torch.zeros(B, V, device=dev), tg.params_to_device(params, dev), torch.zeros(B, device=dev),
                   vocab=V, debug={"post_logits": post})
    torch.cuda.synchronize()
    got = (post == 0).cpu().numpy()
    np.testing.assert_array_equal(got, table_bits(sampler, rows, V), err_msg="table words differ from the sampler's view")
    return got


def make_constraint(sampler, text, toks, eos=-1, n_rows=256):
    from tinygpt_amd import json_schema as J

    V = len(toks)
    sampler.set_mask_table(np.zeros((n_rows, (V + 31) // 32), np.uint32), V)
    return J.JsonSchemaConstraint(sampler, J.schema_from_json(text), toks, eos=eos, n_rows=n_rows)


def test_masker_kats_on_device(sampler):
    """Only '{' at the start of an object schema; a complete automaton
    masks everything, or allows only EOS."""
    from tinygpt_amd import json_schema as J

    toks = U.byte_vocab()
    text = '{ "type": "object", "properties": {}, "required": [] }'
    log("json kats: byte vocabulary, object start")
    c = make_constraint(sampler, text, toks)
    r = c.rows_for([c.start()])
    got = read_rows(sampler, r, 256)[0]
    np.testing.assert_array_equal(got, O.masker_row(O.FSM(O.from_json(text)), toks))
    assert got[ord("{")] and got.sum() == 1
    for eos in (-1, 42):
        log(f"json kats: complete automaton, eos {eos}")
        c = make_constraint(sampler, '{"type":"boolean"}', toks, eos=eos)
        s = J.JsonSchemaFSM.accept_bytes(c.start(), b"true")
        got = read_rows(sampler, c.rows_for([s]), 256)[0]
        of = O.FSM({"t": "boolean"})
        assert of.accept_string("true")
        np.testing.assert_array_equal(got, O.masker_row(of, toks, eos=None if eos < 0 else eos))
        assert got.sum() == (0 if eos < 0 else 1)


@pytest.mark.parametrize("si", range(len(U.FIXTURES) + len(U.EXTRA_SCHEMAS)))
def test_rows_equal_token_replay(sampler, si):
    """Rows of snapshots along random documents (one device call per batch
    of new snapshots) equal the oracle's per-token replay."""
    text = (U.fixture_text(U.FIXTURES[si]) if si < len(U.FIXTURES) else U.EXTRA_SCHEMAS[si - len(U.FIXTURES)])
    toks = U.json_vocab()
    V = len(toks)
    eos = V - 1
    c = make_constraint(sampler, text, toks, eos=eos)
    g = np.random.default_rng(500 + si)
    checked = 0
    for doc in range(2):
        data, snaps = U.random_document(c.fsm, g, max_steps=300, partial=True)
        picks = sorted(set(g.choice(len(snaps), size=min(6, len(snaps)), replace=False).tolist()) | {0, len(snaps) - 1})
        log(f"json rows: schema {si} doc {doc} len {len(data)} snapshots {len(picks)}")
        rows = c.rows_for([snaps[i] for i in picks])
        got = read_rows(sampler, rows, V)
        for k, i in enumerate(picks):
            of = O.FSM(O.from_json(text))
            assert of.accept_bytes(data[:i])
            np.testing.assert_array_equal(got[k], O.masker_row(of, toks, eos=eos),
                                          err_msg=f"schema {si} prefix {data[:i]!r}")
            checked += 1
    assert checked >= 4


def test_constrained_decoding_loop(sampler):
    """Eight sequences decode under pace-fm-label-response: rows for the
    batch's snapshots, one sampling call, commit.  Every sampled token is
    one the oracle's masker allows; every completed document is JSON of
    the schema's shape, and then only EOS is sampled."""
    import torch

    import tinygpt_amd as tg
    from tinygpt_amd import json_schema as J

    text = U.fixture_text("pace-fm-label-response")
    toks = U.json_vocab()
    V = len(toks)
    eos = V - 1
    c = make_constraint(sampler, text, toks, eos=eos, n_rows=2048)
    B = 8
    g = np.random.default_rng(9)

    def utf8(t):
        try:
            t.decode("utf-8")
            return True
        except UnicodeDecodeError:
            return False

    # closing tokens likelier; tokens that are not UTF-8 never sampled
    bias = np.array([(4.0 if (b'"' in t or b"}" in t) else 0.0) if utf8(t) else -np.inf for t in toks], np.float32)
    snaps = [c.start()] * B
    ofs = [O.FSM(O.from_json(text)) for _ in range(B)]
    docs = [bytearray() for _ in range(B)]
    done = [False] * B
    dev = "cuda:0"
    for step in range(160):
        rows = c.rows_for(snaps)
        params = tg.make_params(B, temperature=1.0, top_p=0.95, mask_state=rows.tolist())
        logits = torch.from_numpy(g.standard_normal((B, V)).astype(np.float32) + bias).to(dev)
        u = torch.from_numpy(g.random(B).astype(np.float32)).to(dev)
        ids = sampler.sample(logits, tg.params_to_device(params, dev), u, vocab=V,
                             hint=tg.batch_hint(params, V)).cpu().numpy()
        for b in range(B):
            # the oracle's masker allows the sampled token: EOS once complete,
            # else a non-empty token whose bytes its automaton accepts
            t = int(ids[b])
            assert 0 <= t < V, f"step {step} row {b} id {t}"
            if done[b]:
                assert t == eos and ofs[b].is_complete
                continue
            assert not ofs[b].is_complete and len(toks[t]) > 0 and ofs[b].accept_bytes(toks[t]), \
                f"step {step} row {b} id {t}"
            n = c.commit(snaps[b], int(ids[b]))
            assert n is not None
            snaps[b] = n
            docs[b] += toks[ids[b]]
            done[b] = J.JsonSchemaFSM.is_complete(n)
        if all(done):
            break
    log(f"json decode: {sum(done)} of {B} complete, {c.built} rows built")
    assert sum(done) >= 1
    for b in range(B):
        if done[b]:
            v = json.loads(bytes(docs[b]))
            assert set(v) == {"spokenText", "pointAtLabel", "clickLabel"}
            assert all(isinstance(x, str) for x in v.values())
