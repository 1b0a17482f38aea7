"""The JSON-schema grammar rows on the CPU: the product's automaton
(tinygpt_amd/json_schema.py) and the oracle's independent restatement
(oracle/json_fsm.py) against the reference's known-answer tests
(native-mac/Tests/TinyGPTModelTests/ConstrainedGenTests.swift:12-270), each
other on random byte streams, Python's json module on every complete
document of the reference's schemas (grammars/*.schema.json, copied under
tests/golden/grammars), and the local device DFA against the per-token
replay of LogitsMasker.mask (ConstrainedGen.swift:805-822)."""
import json

import numpy as np
import pytest

import json_fsm as O
import json_schema_util as U
from tinygpt_amd import json_schema as J


class Product:
    """The product automaton behind the reference's mutable interface: a
    rejected byte or byte string leaves the snapshot as it was."""

    def __init__(self, node):
        self.fsm = J.JsonSchemaFSM(node)
        self.s = self.fsm.start

    def accept_byte(self, b):
        n = J.JsonSchemaFSM.accept_byte(self.s, b)
        if n is None:
            return False
        self.s = n
        return True

    def accept_string(self, text):
        n = J.JsonSchemaFSM.accept_bytes(self.s, text.encode())
        if n is None:
            return False
        self.s = n
        return True

    @property
    def is_complete(self):
        return J.JsonSchemaFSM.is_complete(self.s)


def both(schema_text=None, node=None):
    """(product, oracle) automata over the same schema."""
    if schema_text is not None:
        return Product(J.schema_from_json(schema_text)), O.FSM(O.from_json(schema_text))
    return Product(node[0]), O.FSM(node[1])


# ---------------------------------------------------------------- schema parse (:12-45)
def test_parses_object_with_required_and_properties():
    text = '{"type": "object", "required": ["name"], "properties": {"name": {"type": "string"}}}'
    n = J.schema_from_json(text)
    assert n.kind == "object" and len(n.props) == 1 and n.props[0][0] == "name" and "name" in n.required
    o = O.from_json(text)
    assert o["t"] == "object" and [k for k, _ in o["props"]] == ["name"] and "name" in o["req"]


def test_parses_enum_string():
    text = '{ "type": "string", "enum": ["a", "b", "c"] }'
    n = J.schema_from_json(text)
    assert n.kind == "string" and n.enum == ("a", "b", "c")
    assert O.from_json(text)["enum"] == ["a", "b", "c"]


def test_unsupported_shapes_are_any():
    for text in ('{"oneOf": [{"type": "string"}]}', '{"type": "wat"}', '[1]', '{"enum": [1, 2]}'):
        assert J.schema_from_json(text).kind == "any"
        assert O.from_json(text)["t"] == "any"


# ---------------------------------------------------------------- automaton KATs (:48-224)
SIMPLE = '{"type": "object", "properties": {"name": {"type": "string"}, "age": {"type": "integer"}}, "required": ["name", "age"]}'
X_INT = '{ "type": "object", "properties": { "x": { "type": "integer" } }, "required": ["x"] }'


@pytest.mark.parametrize("impl", [0, 1])
def test_fsm_kats(impl):
    def f(text=None, node=None):
        return both(text, node)[impl]

    string_node = (J.SchemaNode("string"), {"t": "string", "enum": None, "min": None, "max": None})
    bool_node = (J.SchemaNode("boolean"), {"t": "boolean"})
    null_node = (J.SchemaNode("null"), {"t": "null"})

    a = f(SIMPLE)  # test_fsmAcceptsSimpleObject
    assert a.accept_string('{"name":"Alice","age":42}') and a.is_complete
    assert not f(X_INT).accept_string('  {"x":1}')  # test_fsmRejectsInterTokenWhitespace
    a = f(node=string_node)  # test_fsmStringAllowsWhitespaceInContent
    assert a.accept_string('"hello world"') and a.is_complete
    a = f(X_INT)  # test_fsmRejectsInvalidJSON
    assert not a.accept_string("garbage") and not a.is_complete
    a = f('{ "type": "object", "properties": { "x": { "type": "integer" } }, "required": [] }')
    assert a.accept_string('{"') and not a.accept_byte(ord("y"))  # test_fsmRejectsUndeclaredKey
    a = f('{ "type": "string", "enum": ["foo", "bar"] }')  # test_fsmEnumRestrictsContent
    assert a.accept_string('"foo"') and a.is_complete
    a = f('{ "type": "string", "enum": ["foo", "bar"] }')  # test_fsmEnumRejectsNonMember
    assert a.accept_string('"') and a.accept_string("f") and not a.accept_byte(ord("x"))
    assert a.accept_string('oo"') and a.is_complete
    a = f('{ "type": "array", "items": { "type": "integer" } }')  # test_fsmAcceptsArray
    assert a.accept_string("[1,2,3]") and a.is_complete
    a = f('{"type": "object", "properties": {"tool_name": {"type": "string", "enum": ["read_file", "run_test"]},'
          '"arguments": {"type": "object", "properties": {"path": {"type": "string"}}}},'
          '"required": ["tool_name", "arguments"]}')  # test_fsmAcceptsNestedObject
    assert a.accept_string('{"tool_name":"read_file","arguments":{"path":"/etc/passwd"}}') and a.is_complete
    for lit, node in (("true", bool_node), ("false", bool_node), ("null", null_node)):  # test_fsmAcceptsBooleansAndNull
        a = f(node=node)
        assert a.accept_string(lit) and a.is_complete
    a = f('{ "type": "object", "properties": { "a": { "type": "integer" }, "b": { "type": "integer" } }, "required": [] }')
    assert a.accept_string('{"a":1') and a.accept_byte(ord(",")) and not a.accept_byte(ord("}"))  # trailing comma
    a = f('{ "type": "array", "items": { "type": "integer" } }')
    assert a.accept_string("[1,2") and a.accept_byte(ord(",")) and not a.accept_byte(ord("]"))
    a = f('{"type": "object", "properties": {"a": {"type": "integer"}, "b": {"type": "integer"}}, "required": ["a", "b"]}')
    assert a.accept_string('{"a":1') and not a.accept_byte(ord("}"))  # test_fsmRequiresAllRequiredKeys
    assert a.accept_string(',"b":2}') and a.is_complete


@pytest.mark.parametrize("impl", [0, 1])
def test_fsm_rules_beyond_the_kats(impl):
    """Rules the reference states in code: escapes (\\uXXXX included) count
    as characters toward maxLength; enums reject backslashes; integers take
    no fraction or exponent; a number ends only at a structural byte, so a
    number at the top level never completes; keys of a fully emitted object
    cannot reopen."""
    f = lambda text: both(text)[impl]
    a = f('{"type":"string","maxLength":3}')
    assert a.accept_string('"\\n') and a.accept_string("a") and not a.accept_byte(ord("b"))
    a = f('{"type":"string","maxLength":6}')
    assert a.accept_string('"\\u00e9"') and a.is_complete
    a = f('{"type":"string","maxLength":5}')
    assert a.accept_string('"\\u00e') and not a.accept_byte(ord("9"))
    assert not f('{"type":"string","enum":["a"]}').accept_string('"\\')
    a = f('{"type":"array","items":{"type":"integer"}}')
    assert a.accept_string("[1") and not a.accept_byte(ord(".")) and not a.accept_byte(ord("e"))
    a = f('{"type":"number"}')
    assert a.accept_string("-0.5e+3") and not a.is_complete and not a.accept_byte(ord(","))
    a = f('{"type":"object","properties":{"a":{"type":"null"}}}')
    assert a.accept_string('{"a":null') and not a.accept_byte(ord(","))
    a = f('{"type":"string","minLength":2}')
    assert a.accept_string('"a') and not a.accept_byte(ord('"'))
    a = f('{"type":"object","required":["k"]}')
    assert a.accept_string('{"z":[1,{"q":true}]') and not a.accept_byte(ord("}"))
    assert a.accept_string(',"k":"v"}') and a.is_complete


def _random_bytes(g, n):
    alphabet = b'{}[]":,-0123456789.eE+tfrulnsab\\/u\x00 \xc3\xa9xyzABF'
    return bytes(g.choice(list(alphabet), n))


SCHEMAS = [U.fixture_text(n) for n in U.FIXTURES] + U.EXTRA_SCHEMAS


@pytest.mark.parametrize("si", range(len(SCHEMAS)))
def test_product_equals_oracle_on_byte_streams(si):
    """Byte by byte, accept / reject and completeness agree, along random
    documents and along random byte streams (a rejected byte is skipped)."""
    text = SCHEMAS[si]
    g = np.random.default_rng(100 + si)
    p, o = both(text)
    for _ in range(40):
        r = U.random_document(p.fsm, g, ascii_only=bool(g.integers(0, 2)))
        if r is None:
            continue
        data, _ = r
        p, o = both(text)
        for b in data:
            assert p.accept_byte(b) == o.accept_byte(b) is True
            assert p.is_complete == o.is_complete
    for trial in range(60):
        # acceptBytes of one byte (restores on rejection, as the masker and
        # commit do; the reference's acceptByte can leave a partly popped
        # stack behind a rejected byte)
        p, o = both(text)
        for b in _random_bytes(g, 200):
            assert p.accept_byte(b) == o.accept_bytes(bytes([b]))
            assert p.is_complete == o.is_complete


# ---------------------------------------------------------------- complete documents are JSON
def _check_value(v, node, raw):
    k = node.kind
    if k == "any":
        return
    if k == "object":
        assert isinstance(v, dict)
        assert node.required <= set(v)
        if node.props:
            assert set(v) <= {n for n, _ in node.props}
        for name, sub in node.props:
            if name in v:
                _check_value(v[name], sub, raw)
    elif k == "string":
        assert isinstance(v, str)
        if node.enum is not None:
            assert v in node.enum
        if node.max_len is not None:
            assert len(v) <= node.max_len  # escapes only shorten the decoded text
    elif k == "number":
        assert isinstance(v, int if node.integer else (int, float)) and not isinstance(v, bool)
    elif k == "boolean":
        assert isinstance(v, bool)
    elif k == "null":
        assert v is None
    elif k == "array":
        assert isinstance(v, list)
        for x in v:
            _check_value(x, node.items, raw)


@pytest.mark.parametrize("name", U.FIXTURES)
def test_complete_documents_are_valid_json(name):
    """Every document the automaton completes on a reference schema parses
    with Python's json module and meets the schema's supported constraints."""
    node = J.schema_from_json(U.fixture_text(name))
    fsm = J.JsonSchemaFSM(node)
    g = np.random.default_rng(len(name))
    done = 0
    for _ in range(80):
        r = U.random_document(fsm, g)
        if r is None:
            continue
        data, _ = r
        v = json.loads(data)
        _check_value(v, node, data)
        done += 1
    assert done >= 40


# ---------------------------------------------------------------- masks (:228-270 and replay)
def test_masker_kats_through_the_automaton():
    """ConstrainedGenTests.swift:228-270 through the automaton: the local
    DFA's row (the device kernel's contract) and the oracle's per-token
    replay on the byte-level vocabulary."""
    toks = U.byte_vocab()
    trie = J.TokenTrie(toks)
    # only '{' at the start of an object schema; whitespace rejected
    text = '{ "type": "object", "properties": {}, "required": [] }'
    node = J.schema_from_json(text)
    d = J.local_dfa([J.JsonSchemaFSM(node).start], trie)
    row = U.dfa_row(d, d.roots[0], toks)
    orow = np.array(O.masker_row(O.FSM(O.from_json(text)), toks))
    np.testing.assert_array_equal(row, orow)
    assert row[ord("{")] and not row[ord(" ")] and not row[ord("a")] and not row[ord("9")]
    assert row.sum() == 1
    # a complete automaton masks everything without EOS, allows only EOS with one
    s = J.JsonSchemaFSM.accept_bytes(J.JsonSchemaFSM(J.SchemaNode("boolean")).start, b"true")
    assert J.JsonSchemaFSM.is_complete(s)
    d = J.local_dfa([s], trie)
    assert not U.dfa_row(d, d.roots[0], toks).any()
    row = U.dfa_row(d, d.roots[0], toks, eos=42)
    assert row[42] and row.sum() == 1
    of = O.FSM({"t": "boolean"})
    assert of.accept_string("true")
    assert not any(O.masker_row(of, toks))
    assert O.masker_row(of, toks, eos=42) == row.tolist()


@pytest.mark.parametrize("si", range(len(SCHEMAS)))
def test_local_dfa_rows_equal_token_replay(si):
    """For snapshots along random documents, the row the local DFA gives
    every token equals the oracle's clone-and-replay of the token's bytes."""
    text = SCHEMAS[si]
    toks = U.json_vocab()
    trie = J.TokenTrie(toks)
    node = J.schema_from_json(text)
    fsm = J.JsonSchemaFSM(node)
    g = np.random.default_rng(300 + si)
    checked = 0
    for _ in range(6):
        data, snaps = U.random_document(fsm, g, max_steps=400, partial=True)
        picks = sorted(set(g.choice(len(snaps), size=min(6, len(snaps)), replace=False).tolist()) | {0, len(snaps) - 1})
        d = J.local_dfa([snaps[i] for i in picks], trie)
        for root, i in zip(d.roots, picks):
            of = O.FSM(O.from_json(text))
            assert of.accept_bytes(data[:i])
            np.testing.assert_array_equal(U.dfa_row(d, root, toks, eos=5), np.array(O.masker_row(of, toks, eos=5)),
                                          err_msg=f"schema {si} prefix {data[:i]!r}")
            checked += 1
    assert checked >= 10


@pytest.mark.parametrize("si", range(len(SCHEMAS)))
def test_local_dfa_cache_gives_the_same_automaton(si):
    """local_dfa with a step cache kept across calls (as JsonSchemaConstraint
    keeps it) builds the same automaton as a fresh build: the same
    transitions, completion flags and roots, call after call."""
    text = SCHEMAS[si]
    toks = U.json_vocab()
    trie = J.TokenTrie(toks)
    fsm = J.JsonSchemaFSM(J.schema_from_json(text))
    g = np.random.default_rng(500 + si)
    cache = {}
    for _ in range(4):
        _, snaps = U.random_document(fsm, g, max_steps=300, partial=True)
        picks = sorted(set(g.choice(len(snaps), size=min(8, len(snaps)), replace=False).tolist()))
        want = J.local_dfa([snaps[i] for i in picks], J.TokenTrie(toks))
        got = J.local_dfa([snaps[i] for i in picks], trie, cache=cache)
        np.testing.assert_array_equal(got.trans, want.trans)
        np.testing.assert_array_equal(got.complete, want.complete)
        assert got.roots == want.roots
        # byte classes: equal columns share a class, numbered by first byte
        # (checked against a sort of the columns, np.unique)
        bc, ct = got.byte_classes()
        _, first, inv = np.unique(got.trans.T, axis=0, return_index=True, return_inverse=True)
        rank = np.empty(len(first), dtype=np.int64)
        rank[np.argsort(first)] = np.arange(len(first))
        np.testing.assert_array_equal(bc, rank[inv.reshape(-1)].astype(np.uint8))
        np.testing.assert_array_equal(ct, got.trans[:, np.sort(first)])
    assert cache


def test_canonical_keys_merge_equivalent_snapshots():
    """Free strings of different contents with the same counted length share
    a key; so do any-object keys no required name extends; enum prefixes
    and declared keys stay distinct."""
    node = J.schema_from_json('{"type":"object","properties":{"s":{"type":"string"},"m":{"type":"string","maxLength":4}},'
                              '"required":["s"]}')
    f = J.JsonSchemaFSM(node)
    k = lambda b: J.canonical_key(J.JsonSchemaFSM.accept_bytes(f.start, b))
    assert k(b'{"s":"abc') == k(b'{"s":"xyz') == k(b'{"s":"')
    assert k(b'{"m":"ab') == k(b'{"m":"xy') != k(b'{"m":"abc')
    assert k(b'{"s') != k(b'{"m')
    node = J.schema_from_json('{"type":"object","required":["ab"]}')
    f = J.JsonSchemaFSM(node)
    assert k(b'{"zz') == k(b'{"qq') != k(b'{"a')
    assert k(b'{"zz":1') == k(b'{"qq":1') != k(b'{"ab":1')


@pytest.mark.parametrize("si", range(len(SCHEMAS)))
def test_row_keys_share_only_equal_rows(si):
    """Snapshots that share a row key (an open string's count kept only as
    far as a token can see it) get equal rows; along a long string the keys
    collapse to a few."""
    text = SCHEMAS[si]
    toks = U.json_vocab(n_random=300)
    trie = J.TokenTrie(toks)
    fsm = J.JsonSchemaFSM(J.schema_from_json(text))
    g = np.random.default_rng(700 + si)
    snaps = []
    for _ in range(4):
        _, sn = U.random_document(fsm, g, max_steps=300, partial=True)
        snaps += sn
    d = J.local_dfa(snaps, trie)
    by_key = {}
    for s, root in zip(snaps, d.roots):
        row = U.dfa_row(d, root, toks, eos=3)
        k = J.row_key(s, trie.max_len)
        if k in by_key:
            np.testing.assert_array_equal(by_key[k], row)
        else:
            by_key[k] = row
    assert len(by_key) <= len(set(J.canonical_key(s) for s in snaps))


def test_row_keys_collapse_a_long_string():
    f = J.JsonSchemaFSM(J.schema_from_json(U.fixture_text("pace-fm-response-v11")))
    s = J.JsonSchemaFSM.accept_bytes(f.start, b'{"spokenText":"')
    keys = set()
    for _ in range(400):  # counts 0 .. 399 of maxLength 400
        keys.add(J.row_key(s, 24))
        s = J.JsonSchemaFSM.accept_byte(s, ord("a"))
    assert J.JsonSchemaFSM.accept_byte(s, ord("a")) is None  # a 401st character is refused
    # count 0 (one more needed before the quote), counts 1..375 (room beyond any token), then 376..399
    assert len(keys) == 26
