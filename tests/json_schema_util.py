"""Shared helpers of the JSON-schema tests: the fixture schemas, a
JSON-ish test vocabulary, random documents walked through the automaton,
and the mask-row contract of tgs_mask_rows_from_dfa applied to a local DFA
on the CPU."""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GRAMMARS = os.path.join(HERE, "golden", "grammars")
FIXTURES = ["pace-fm-response", "pace-fm-label-response", "pace-fm-label-response-v9", "pace-fm-response-v10",
            "pace-fm-response-v11"]


def fixture_text(name):
    with open(os.path.join(GRAMMARS, name + ".schema.json")) as f:
        return f.read()


# schemas exercising what the fixtures leave out: nested arrays, numbers,
# escapes, enums with shared prefixes, keys of an object without declared
# properties but with required names, booleans and null
EXTRA_SCHEMAS = [
    '{"type":"object","properties":{"tool_name":{"type":"string","enum":["read_file","run_test","read"]},'
    '"arguments":{"type":"object","properties":{"path":{"type":"string"}}}},"required":["tool_name","arguments"]}',
    '{"type":"array","items":{"type":"object","properties":{"x":{"type":"number"},"ok":{"type":"boolean"},'
    '"n":{"type":"null"},"t":{"type":"string","maxLength":5}},"required":["x"]}}',
    '{"type":"object","required":["ab","b"]}',
    '{"type":"object","properties":{"v":{}, "s":{"type":"string","minLength":2,"maxLength":9}},"required":["s"]}',
    '{"type":"array","items":{"type":"array","items":{"type":"integer"}}}',
]


def byte_vocab():
    """Token i = the bytes of String(decoding: [UInt8(i)], as: UTF8.self):
    the byte itself below 0x80, U+FFFD (EF BF BD) for a lone high byte
    (ConstrainedGenTests.swift:232-235)."""
    return [bytes([i]) if i < 0x80 else b"\xef\xbf\xbd" for i in range(256)]


def json_vocab(n_random=1500, seed=7):
    """Single bytes, JSON structural pieces, keys and values of the
    fixtures, escapes, numbers and random text pieces (some with quotes,
    backslashes or multi-byte UTF-8)."""
    g = np.random.default_rng(seed)
    toks = [bytes([i]) for i in range(256)]
    pieces = ['{"', '"}', '":"', '","', '":', '",', '},', '},{', '[{', '}]', '[[', ']]', '],[', '[]', '{}', '""',
              '":{"', '":[', 'true', 'false', 'null', 'tru', 'nul', '\\n', '\\"', '\\u00', '\\u', '\\\\', '0.5', '-1',
              '12', '1e', 'e+', '.25', '00', 'spokenText', '"spokenText":"', 'intent', '"intent":"', 'action',
              'answer', 'payload', '"payload":{', 'args', 'calls', 'name', 'text', 'pointAtElementId',
              'clickElementId', 'pointAtLabel', 'clickLabel', 'bodyText', 'read_file', 'run_test', 'read', 'path',
              'tool_name', 'arguments', '"x":', '"ok":', '"t":"', ' hello', ' world', 'Hi', '!', '?', 'é', '—', '...',
              ' the', '"ab":', '"b":', 'ab', '":1}', '":1,"', ':-', '1}', '1]', '2,', '],', '}}', '"}}', '"},"',
              'clarify', 'confirm_destructive', 'out_of_scope', 'dictate', 'edit', '"reference":"', '"name":"']
    toks += [p.encode() for p in pieces]
    alphabet = list('abcdefghijklmnopqrstuvwxyz ABCDE.,:;"{}[]\\0123456789-_é')
    for _ in range(n_random):
        n = int(g.integers(1, 16))
        toks.append("".join(g.choice(alphabet, n)).encode())
    toks.append(b" " * 24)
    toks.append(b"")  # an empty token: never allowed
    return toks


def dfa_row(dfa, root, tokens, eos=-1):
    """The row tgs_mask_rows_from_dfa writes for DFA state root: a token is
    allowed when non-empty and every byte has a transition; a complete
    state allows only EOS."""
    if dfa.complete[root]:
        row = np.zeros(len(tokens), dtype=bool)
        if 0 <= eos < len(tokens):
            row[eos] = True
        return row
    return np.array([len(t) > 0 and dfa.walk(root, t) >= 0 for t in tokens], dtype=bool)


def random_document(fsm, g, max_steps=3000, ascii_only=True, partial=False):
    """Bytes walked from the start snapshot, each chosen among the bytes the
    automaton accepts (printable ASCII when ascii_only), closing bytes ever
    more likely, until the snapshot is complete; returns (data, snapshots
    along the way), or None when the walk runs too long (partial: the walk
    so far)."""
    from tinygpt_amd.json_schema import JsonSchemaFSM

    s = fsm.start
    out = bytearray()
    snaps = [s]
    cand = list(range(0x20, 0x7F)) if ascii_only else list(range(256))
    closers = set(b'"}]0123456789el')
    for step in range(max_steps):
        if JsonSchemaFSM.is_complete(s):
            return bytes(out), snaps
        ok = [(b, n) for b in cand if (n := JsonSchemaFSM.accept_byte(s, b)) is not None]
        if not ok:
            return (bytes(out), snaps) if partial else None
        w = np.array([1.0 + (step / 20.0 if b in closers else 0.0) for b, _ in ok])
        b, n = ok[int(g.choice(len(ok), p=w / w.sum()))]
        out.append(b)
        s = n
        snaps.append(s)
    return (bytes(out), snaps) if partial else None
