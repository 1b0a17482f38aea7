"""JSON-schema constrained decoding on the device mask table.

The host side of the reference's JSON-schema grammar rows, restated:

* `parse_schema` -- the Draft-7 subset of JSONSchemaNode.from(data:)
  (native-mac/Sources/TinyGPTModel/JSONSchema.swift:40-117);
* `JsonSchemaFSM` -- JSONSchemaFSM, the byte-level pushdown automaton
  (native-mac/Sources/TinyGPTModel/ConstrainedGen.swift:35-749): a frame
  stack, minified JSON only, required-key gating, enum prefix pruning, a
  depth cap of 64 nested re-feeds.  Snapshots are immutable tuples, so a
  snapshot is its own clone;
* `local_dfa` -- the device form of one or more snapshots: every state the
  automaton reaches from them within the longest token's byte length,
  interned by a canonical key (parts of a snapshot that cannot change any
  later decision are dropped from the key: the content of a free string
  beyond what its length limits count, the text of keys no required set
  can name), as a byte-level DFA that tgs_mask_rows_from_dfa replays every
  token through.  A token is allowed exactly when each of its bytes is
  accepted from the snapshot (LogitsMasker.mask(forFSM:),
  ConstrainedGen.swift:805-822); a complete snapshot allows only EOS;
* `JsonSchemaConstraint` -- per-sequence snapshots interned as rows of the
  sampler's mask table, new rows built on the device in one call per batch,
  and commit of the sampled token (LogitsMasker.commit,
  ConstrainedGen.swift:827-830).

String contents follow the reference: each body byte appends one
character (the byte read as a Latin-1 code point), an escape appends its
two characters (\\uXXXX: six), and length limits count those characters.
"""
from __future__ import annotations

import contextlib
import json

import numpy as np

__all__ = ["SchemaNode", "parse_schema", "schema_from_json", "JsonSchemaFSM", "TokenTrie", "local_dfa", "LocalDfa",
           "JsonSchemaConstraint"]


# ------------------------------------------------------------------ schema
class SchemaNode:
    """One node of the supported schema subset.  kind: object, string,
    number, boolean, null, array or any."""

    __slots__ = ("kind", "props", "required", "enum", "min_len", "max_len", "integer", "items")

    def __init__(self, kind, props=(), required=frozenset(), enum=None, min_len=None, max_len=None,
                 integer=False, items=None):
        self.kind = kind
        self.props = tuple(props)
        self.required = frozenset(required)
        self.enum = None if enum is None else tuple(enum)
        self.min_len = min_len
        self.max_len = max_len
        self.integer = integer
        self.items = items

    def __repr__(self):
        return f"SchemaNode({self.kind})"


ANY = SchemaNode("any")
ANY_OBJECT = SchemaNode("object")  # the object an `any` value opens: no declared keys


def _int_or_none(v):
    # JSONSerialization numbers bridge to Int only when integral
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    if isinstance(v, float) and not v.is_integer():
        return None
    return int(v)


def parse_schema(obj) -> SchemaNode:
    """JSONSchemaNode.parse (JSONSchema.swift:72-116): unsupported shapes
    become `any`; `enum` with string members wins over `type`; object
    properties are ordered by key."""
    if not isinstance(obj, dict):
        return ANY
    en = obj.get("enum")
    if isinstance(en, list):
        strings = [e for e in en if isinstance(e, str)]
        if strings:
            return SchemaNode("string", enum=strings, min_len=_int_or_none(obj.get("minLength")),
                              max_len=_int_or_none(obj.get("maxLength")))
    t = obj.get("type")
    if not isinstance(t, str):
        return ANY
    if t == "object":
        raw = obj.get("properties")
        raw = raw if isinstance(raw, dict) else {}
        props = [(k, parse_schema(raw[k])) for k in sorted(raw)]
        req = obj.get("required")
        req = [r for r in req if isinstance(r, str)] if isinstance(req, list) and all(isinstance(r, str) for r in req) else []
        return SchemaNode("object", props=props, required=req)
    if t == "string":
        return SchemaNode("string", min_len=_int_or_none(obj.get("minLength")), max_len=_int_or_none(obj.get("maxLength")))
    if t == "number":
        return SchemaNode("number", integer=False)
    if t == "integer":
        return SchemaNode("number", integer=True)
    if t == "boolean":
        return SchemaNode("boolean")
    if t == "null":
        return SchemaNode("null")
    if t == "array":
        return SchemaNode("array", items=parse_schema(obj.get("items")))
    return ANY


def schema_from_json(text) -> SchemaNode:
    """JSONSchemaNode.from(data:) over schema text (str or bytes)."""
    return parse_schema(json.loads(text))


# ------------------------------------------------------------------ automaton
# Frames (tuples, tag first):
#   ("V", node, done)                          value slot
#   ("O", node, emitted, phase, key)           object
#   ("A", items, phase)                        array
#   ("S", st, digits, enum, min, max, content, is_key)   string
#   ("N", st, integer)                         number
#   ("T", literal, position)                   true / false
#   ("Z", position)                            null
O_OPEN, O_COMMA, O_KEY, O_VALUE, O_AFTER, O_CLOSED = range(6)
A_OPEN, A_COMMA, A_ITEM, A_CLOSED = range(4)
S_BODY, S_ESC, S_UNI, S_CLOSED = range(4)
N_SIGN, N_ZERO, N_INT, N_POINT, N_FRAC, N_EXP, N_EXPSIGN, N_EXPDIG = range(8)
_N_ACCEPTING = (N_ZERO, N_INT, N_FRAC, N_EXPDIG)

# transition actions (ConstrainedGen.swift:130-160)
_REJECT, _REPLACE, _PUSH, _REPLACE_PUSH, _PUSH_RETRY, _POP, _POP_RETRY = range(7)
_REJ = (_REJECT,)

_DIGITS = frozenset(b"0123456789")
_HEX = frozenset(b"0123456789abcdefABCDEF")
_ESCAPES = frozenset(b'"\\/bfnrt')
_TERMS = frozenset(b",}] \t\n\r")
MAX_REFEED = 64  # driveByte's depth cap


def _new_string(enum=None, min_len=None, max_len=None, is_key=False):
    return ("S", S_BODY, 0, enum, min_len, max_len, "", is_key)


def _open_value(node, b):
    k = node.kind
    if k == "any":
        if b == 0x7B:  # {
            return (_PUSH, ("O", ANY_OBJECT, frozenset(), O_OPEN, None))
        if b == 0x5B:  # [
            return (_PUSH, ("A", ANY, A_OPEN))
        if b == 0x22:
            return (_PUSH, _new_string())
        if b == 0x2D:  # -
            return (_PUSH, ("N", N_SIGN, False))
        if b == 0x74:  # t
            return (_PUSH, ("T", "true", 1))
        if b == 0x66:  # f
            return (_PUSH, ("T", "false", 1))
        if b == 0x6E:  # n
            return (_PUSH, ("Z", 1))
        if b in _DIGITS:
            return (_PUSH, ("N", N_ZERO if b == 0x30 else N_INT, False))
        return _REJ
    if k == "object":
        return (_PUSH, ("O", node, frozenset(), O_OPEN, None)) if b == 0x7B else _REJ
    if k == "array":
        return (_PUSH, ("A", node.items, A_OPEN)) if b == 0x5B else _REJ
    if k == "string":
        return (_PUSH, _new_string(node.enum, node.min_len, node.max_len)) if b == 0x22 else _REJ
    if k == "number":
        if b == 0x2D:
            return (_PUSH, ("N", N_SIGN, node.integer))
        if b in _DIGITS:
            return (_PUSH, ("N", N_ZERO if b == 0x30 else N_INT, node.integer))
        return _REJ
    if k == "boolean":
        if b == 0x74:
            return (_PUSH, ("T", "true", 1))
        if b == 0x66:
            return (_PUSH, ("T", "false", 1))
        return _REJ
    if k == "null":
        return (_PUSH, ("Z", 1)) if b == 0x6E else _REJ
    return _REJ


def _unemitted_keys(node, emitted):
    """Declared keys not yet emitted; None for objects without declared keys."""
    if node.kind == "object":
        if not node.props:
            return None
        return tuple(k for k, _ in node.props if k not in emitted)
    return None


def _schema_for(key, node):
    if node.kind == "object":
        for k, v in node.props:
            if k == key:
                return v
    return ANY


def _closable(node, emitted):
    return node.kind != "object" or node.required <= emitted


def _step_object(f, b):
    _, node, emitted, phase, key = f
    if phase == O_OPEN or phase == O_COMMA:
        if phase == O_OPEN and b == 0x7D:  # } (empty object)
            return (_POP,) if _closable(node, emitted) else _REJ
        if b == 0x22:
            keys = _unemitted_keys(node, emitted)
            if keys is not None and not keys:
                return _REJ
            return (_PUSH, _new_string(enum=keys, is_key=True))
        return _REJ
    if phase == O_KEY:
        if b == 0x3A:  # :
            return (_REPLACE_PUSH, ("O", node, emitted, O_VALUE, key), ("V", _schema_for(key, node), False))
        return _REJ
    if phase == O_AFTER:
        if b == 0x2C:  # ,
            rem = _unemitted_keys(node, emitted)
            if rem is not None and not rem:
                return _REJ
            return (_REPLACE, ("O", node, emitted, O_COMMA, key))
        if b == 0x7D:
            return (_POP,) if _closable(node, emitted) else _REJ
        return _REJ
    return _REJ  # inside a value (bytes go to the child) or closed


def _step_array(f, b):
    _, items, phase = f
    if phase == A_OPEN:
        if b == 0x5D:  # ]
            return (_POP,)
        return (_PUSH_RETRY, ("V", items, False))
    if phase == A_COMMA:
        return (_PUSH_RETRY, ("V", items, False))
    if phase == A_ITEM:
        if b == 0x2C:
            return (_REPLACE, ("A", items, A_COMMA))
        if b == 0x5D:
            return (_POP,)
    return _REJ


_PREFIX_SETS = {}


def _prefixes(names):
    """Every prefix of every string of names (a tuple or frozenset), as a
    set, built once per collection: s is a prefix of some member exactly when
    s is in it."""
    p = _PREFIX_SETS.get(names)
    if p is None:
        if len(_PREFIX_SETS) > 100000:
            _PREFIX_SETS.clear()
        p = _PREFIX_SETS[names] = frozenset(e[:i] for e in names for i in range(len(e) + 1))
    return p


def _step_string(f, b):
    _, st, digits, enum, mn, mx, content, is_key = f
    if st == S_BODY:
        if b == 0x22:
            if enum is not None and content not in enum:
                return _REJ
            if mn is not None and len(content) < mn:
                return _REJ
            return (_POP,)
        if b == 0x5C:  # backslash
            if enum is not None:
                return _REJ
            return (_REPLACE, ("S", S_ESC, 0, enum, mn, mx, content, is_key))
        if b < 0x20:
            return _REJ
        nc = content + chr(b)
        if mx is not None and len(nc) > mx:
            return _REJ
        if enum is not None and nc not in _prefixes(enum):
            return _REJ
        return (_REPLACE, ("S", S_BODY, 0, enum, mn, mx, nc, is_key))
    if st == S_ESC:
        if b in _ESCAPES:
            nc = content + "\\" + chr(b)
            if mx is not None and len(nc) > mx:
                return _REJ
            return (_REPLACE, ("S", S_BODY, 0, enum, mn, mx, nc, is_key))
        if b == 0x75:  # u
            nc = content + "\\u"
            if mx is not None and len(nc) > mx:
                return _REJ
            return (_REPLACE, ("S", S_UNI, 0, enum, mn, mx, nc, is_key))
        return _REJ
    if st == S_UNI:
        if b in _HEX:
            nc = content + chr(b)
            if mx is not None and len(nc) > mx:
                return _REJ
            if digits + 1 == 4:
                return (_REPLACE, ("S", S_BODY, 0, enum, mn, mx, nc, is_key))
            return (_REPLACE, ("S", S_UNI, digits + 1, enum, mn, mx, nc, is_key))
        return _REJ
    return _REJ


def _step_number(f, b):
    _, st, integer = f
    if b in _TERMS:
        return (_POP_RETRY,) if st in _N_ACCEPTING else _REJ
    dig = b in _DIGITS
    if st == N_SIGN:
        if b == 0x30:
            return (_REPLACE, ("N", N_ZERO, integer))
        return (_REPLACE, ("N", N_INT, integer)) if dig else _REJ
    if st == N_ZERO or st == N_INT:
        if st == N_INT and dig:
            return (_REPLACE, f)
        if b == 0x2E and not integer:
            return (_REPLACE, ("N", N_POINT, integer))
        if (b == 0x65 or b == 0x45) and not integer:
            return (_REPLACE, ("N", N_EXP, integer))
        return _REJ
    if st == N_POINT:
        return (_REPLACE, ("N", N_FRAC, integer)) if dig else _REJ
    if st == N_FRAC:
        if dig:
            return (_REPLACE, f)
        if b == 0x65 or b == 0x45:
            return (_REPLACE, ("N", N_EXP, integer))
        return _REJ
    if st == N_EXP:
        if b == 0x2B or b == 0x2D:
            return (_REPLACE, ("N", N_EXPSIGN, integer))
        return (_REPLACE, ("N", N_EXPDIG, integer)) if dig else _REJ
    if st == N_EXPSIGN:
        return (_REPLACE, ("N", N_EXPDIG, integer)) if dig else _REJ
    if st == N_EXPDIG:
        return (_REPLACE, f) if dig else _REJ
    return _REJ


def _step_literal(lit, pos, b, make):
    if pos >= len(lit) or b != ord(lit[pos]):
        return _REJ
    if pos + 1 == len(lit):
        return (_POP,)
    return (_REPLACE, make(pos + 1))


def _transition(top, b):
    tag = top[0]
    if tag == "S":
        return _step_string(top, b)
    if tag == "V":
        return _REJ if top[2] else _open_value(top[1], b)
    if tag == "O":
        return _step_object(top, b)
    if tag == "A":
        return _step_array(top, b)
    if tag == "N":
        return _step_number(top, b)
    if tag == "T":
        return _step_literal(top[1], top[2], b, lambda p: ("T", top[1], p))
    if tag == "Z":
        return _step_literal("null", top[1], b, lambda p: ("Z", p))
    return _REJ


def _advance(stack, last_key):
    """advanceParentAfterChildPop (ConstrainedGen.swift:302-347)."""
    while stack:
        p = stack[-1]
        tag = p[0]
        if tag == "O":
            _, node, emitted, phase, key = p
            if phase == O_OPEN or phase == O_COMMA:
                p = ("O", node, emitted, O_KEY, last_key if last_key is not None else "")
            elif phase == O_VALUE:
                p = ("O", node, emitted | {key}, O_AFTER, key)
            return stack[:-1] + (p,)
        if tag == "A":
            return stack[:-1] + (("A", p[1], A_ITEM),)
        if tag == "V":
            if len(stack) == 1:
                return (("V", p[1], True),)
            stack = stack[:-1]
            continue
        return stack
    return stack


def _drive(stack, b, depth=0):
    """driveByte (ConstrainedGen.swift:217-266) on an immutable stack: the
    new stack, or None when the byte is rejected.  Insignificant whitespace
    is never skipped (allowsWhitespaceHere is false everywhere)."""
    if depth > MAX_REFEED or not stack:
        return None
    top = stack[-1]
    act = _transition(top, b)
    k = act[0]
    if k == _REJECT:
        return None
    if k == _REPLACE:
        return stack[:-1] + (act[1],)
    if k == _PUSH:
        return stack + (act[1],)
    if k == _REPLACE_PUSH:
        return stack[:-1] + (act[1], act[2])
    if k == _PUSH_RETRY:
        return _drive(stack + (act[1],), b, depth + 1)
    if k == _POP:
        key = top[6] if top[0] == "S" and top[7] else None
        return _advance(stack[:-1], key)
    # _POP_RETRY
    return _drive(_advance(stack[:-1], None), b, depth + 1)


class JsonSchemaFSM:
    """Snapshots of the automaton: immutable frame stacks.  Methods take and
    return snapshots; None stands for a rejected byte sequence."""

    def __init__(self, root: SchemaNode):
        self.root = root
        self.start = (("V", root, False),)

    @staticmethod
    def accept_byte(snap, b):
        return _drive(snap, b)

    @staticmethod
    def accept_bytes(snap, data):
        """acceptBytes: the snapshot after every byte, or None (the caller's
        snapshot is untouched either way)."""
        s = snap
        for b in data:
            s = _drive(s, b)
            if s is None:
                return None
        return s

    @staticmethod
    def is_complete(snap):
        return len(snap) == 1 and snap[0][0] == "V" and snap[0][2]


# ------------------------------------------------------------------ canonical keys
_OTHER = "\x00<other>"  # a key text no required set contains or extends


def _canon_frame(f, below):
    tag = f[0]
    if tag == "S":
        _, st, digits, enum, mn, mx, content, is_key = f
        if enum is not None:
            c = content
        elif is_key:
            req = below[1].required if below is not None and below[0] == "O" else frozenset()
            c = content if content in _prefixes(req) else _OTHER
        else:
            cap = max(mn or 0, (mx + 1) if mx is not None else 0)
            c = min(len(content), cap)
        return ("S", st, digits, enum, mn, mx, c, is_key)
    if tag == "O":
        _, node, emitted, phase, key = f
        if node.props:
            return f
        req = node.required
        k = key if (key is None or key in req) else _OTHER
        return ("O", node, emitted & req, phase, k)
    return f


def canonical_key(snap):
    """Key under which snapshots with the same future behaviour coincide."""
    out = []
    below = None
    for f in snap:
        out.append(_canon_frame(f, below))
        below = f
    return tuple(out)


_PLAIN = [b for b in range(0x20, 256) if b != 0x22 and b != 0x5C]


def _is_free(snap):
    """Top frame a string body whose plain bytes (0x20 and up, not quote
    or backslash) all lead to one canonical successor: a string without
    enum that is not a key, or a key no required key name extends."""
    top = snap[-1]
    if top[0] != "S" or top[1] != S_BODY or top[3] is not None:
        return False
    if not top[7]:
        return True
    return _canon_frame(top, snap[-2] if len(snap) > 1 else None)[6] == _OTHER


def row_key(snap, max_len: int):
    """Key under which snapshots get the same mask row: the canonical key,
    except that an open free string's character count is kept only as far as
    a token of at most max_len bytes can see it (how many characters the
    string still needs before it may close, and how many it may still take,
    each capped at max_len + 1)."""
    key = canonical_key(snap)
    top = key[-1]
    if top[0] == "S" and isinstance(top[6], int):
        _, st, digits, enum, mn, mx, cnt, is_key = top
        cap = max_len + 1
        need = min(max((mn or 0) - cnt, 0), cap)
        room = cap if mx is None else min(mx - cnt, cap)
        key = key[:-1] + (("S", st, digits, enum, None, None, ("need", need, "room", room), is_key),)
    return key


def _byte_groups(snap):
    """Groups of bytes with the same canonical successor from snap (each
    group evaluated once), as (representative, bytes) pairs; bytes outside
    every group are rejected."""
    top = snap[-1]
    if top[0] == "S":
        _, st, digits, enum, mn, mx, content, is_key = top
        if st == S_BODY and enum is not None:
            # only the next character of an enum member extends the content
            nxt = sorted({ord(e[len(content)]) for e in enum if e.startswith(content) and len(e) > len(content)})
            return [(b, [b]) for b in nxt if 0x20 <= b < 256 and b != 0x22 and b != 0x5C] + [(0x22, [0x22])]
        if st == S_BODY and _is_free(snap):
            return [(0x22, [0x22]), (0x5C, [0x5C]), (0x41, _PLAIN)]
        if not is_key:  # a free string: only counted characters matter
            if st == S_ESC:
                esc = sorted(_ESCAPES)
                return [(esc[0], esc), (0x75, [0x75])]
            if st == S_UNI:
                hx = sorted(_HEX)
                return [(hx[0], hx)]
    return [(b, [b]) for b in range(256)]


class TokenTrie:
    """The vocabulary's byte strings sorted, as a trie of ranges: the
    tokens sharing a prefix of length d are one contiguous range."""

    def __init__(self, tokens):
        toks = [bytes(t) for t in tokens]
        self.max_len = max((len(t) for t in toks), default=0)
        order = sorted(range(len(toks)), key=lambda i: toks[i])
        L = max(self.max_len, 1)
        arr = np.full((len(toks), L), -1, dtype=np.int16)
        for r, i in enumerate(order):
            t = toks[i]
            if t:
                arr[r, :len(t)] = np.frombuffer(t, dtype=np.uint8)
        self.arr = arr
        special = (arr >= 0) & ((arr < 0x20) | (arr == 0x22) | (arr == 0x5C))
        self.last_special = np.where(special, np.arange(L, dtype=np.int16)[None, :], -1).max(axis=1)
        self.n = len(toks)
        self._kids = {}  # (lo, hi, d) -> children: the trie never changes, and walks revisit its nodes
        self._spec = {}  # (lo, hi) -> last depth holding a quote, backslash or control byte

    def children(self, lo, hi, d):
        """(byte, lo, hi) of each child of the node (range [lo, hi), depth d)."""
        key = (lo, hi, d)
        kids = self._kids.get(key)
        if kids is None:
            kids = self._kids[key] = self._children(lo, hi, d)
        return kids

    def last_special_of(self, lo, hi):
        """The deepest quote, backslash or control byte of tokens [lo, hi) (-1: none)."""
        v = self._spec.get((lo, hi))
        if v is None:
            v = self._spec[(lo, hi)] = int(self.last_special[lo:hi].max())
        return v

    def _children(self, lo, hi, d):
        if d >= self.max_len:
            return []
        col = self.arr[lo:hi, d]
        st = int(np.searchsorted(col, 0))  # tokens ending at d sort first (-1)
        if st >= len(col):
            return []
        c = col[st:]
        cuts = np.flatnonzero(np.diff(c)) + 1
        bounds = [0] + cuts.tolist() + [len(c)]
        return [(int(c[bounds[k]]), lo + st + bounds[k], lo + st + bounds[k + 1]) for k in range(len(bounds) - 1)]


class LocalDfa:
    """trans int32 [n, 256] (-1 rejects), complete uint8 [n], roots: the
    state of each requested snapshot, reps: a snapshot per state."""

    def __init__(self, trans, complete, roots, reps):
        self.trans = trans
        self.complete = complete
        self.roots = roots
        self.reps = reps

    @property
    def n(self):
        return self.trans.shape[0]

    def byte_classes(self):
        """(byte_class uint8 [256], trans int32 [n, n_cls]) as tinygpt_amd.grammar.Dfa.byte_classes:
        bytes with equal columns share a class, classes numbered in the order
        of their first byte (columns compared by their bytes, one pass)."""
        cols = np.ascontiguousarray(self.trans.T)
        seen, firsts = {}, []
        byte_class = np.empty(256, dtype=np.uint8)
        for b in range(256):
            c = seen.setdefault(cols[b].tobytes(), len(firsts))
            if c == len(firsts):
                firsts.append(b)
            byte_class[b] = c
        ctrans = np.ascontiguousarray(self.trans[:, firsts], dtype=np.int32)
        return byte_class, ctrans

    def walk(self, state, data):
        """State after data (-1 when a byte is rejected): the walk the device
        kernel makes for one token."""
        s = state
        for b in data:
            s = int(self.trans[s, b])
            if s < 0:
                return -1
        return s


def local_dfa(snaps, trie: TokenTrie, max_states: int = 200000, cache=None) -> LocalDfa:
    """Device form of the snapshots: a byte-level DFA whose walk of every
    vocabulary token from the snapshot's root state rejects exactly when
    the automaton rejects one of the token's bytes.

    States are snapshots interned by canonical key.  The exploration
    follows the vocabulary trie: from a structural state only the bytes
    some token continues with are stepped; a free string body gets its
    whole row at once (three byte groups) along the chain of counted
    characters, and the trie walk under it descends only into subtrees
    holding a quote, a backslash or a control byte.  Transitions no token
    reaches stay -1.  Raises ValueError past max_states.

    cache: a dict kept by the caller across calls, holding each (state key,
    byte) -> (successor key, successor snapshot) step and each state's byte
    groups, so that later calls do not drive the automaton again for steps
    an earlier call took (snapshots of one canonical key behave alike, the
    premise of the interning).  The result is the same with or without it."""
    ids = {}
    reps, rows, done, full, keys = [], [], [], [], []
    chain = []  # free strings: depth of plain bytes whose rows are complete

    def intern(s, key=None):
        if key is None:
            key = canonical_key(s)
        i = ids.get(key)
        if i is None:
            i = len(reps)
            if i >= max_states:
                raise ValueError(f"local automaton exceeds {max_states} states")
            ids[key] = i
            keys.append(key)
            reps.append(s)
            rows.append(np.full(256, -1, dtype=np.int32))
            done.append(np.zeros(256, dtype=bool))
            full.append(False)
            chain.append(0)
        return i

    def step(i, b):
        if not done[i][b]:
            hit = cache.get((keys[i], b)) if cache is not None else None
            if hit is None:
                nxt = _drive(reps[i], b)
                hit = (None, None) if nxt is None else (canonical_key(nxt), nxt)
                if cache is not None:
                    cache[(keys[i], b)] = hit
            rows[i][b] = -1 if hit[0] is None else intern(hit[1], hit[0])
            done[i][b] = True
        return int(rows[i][b])

    def groups(i):
        if cache is None:
            return _byte_groups(reps[i])
        g = cache.get(("groups", keys[i]))
        if g is None:
            g = cache[("groups", keys[i])] = [(r, np.asarray(grp, dtype=np.intp)) for r, grp in _byte_groups(reps[i])]
        return g

    def fill(i):
        if not full[i]:
            for rep, group in groups(i):
                j = step(i, rep)
                rows[i][group] = j
                done[i][group] = True
            full[i] = True

    def ensure_chain(i, rem):
        while rem > 0 and chain[i] < rem and _is_free(reps[i]):
            fill(i)
            chain[i] = rem
            j = int(rows[i][0x41])
            if j < 0:
                break
            i, rem = j, rem - 1

    L = trie.max_len
    roots = [intern(s) for s in snaps]
    for r in roots:
        work = [(r, 0, trie.n, 0)]
        while work:
            i, lo, hi, d = work.pop()
            if d >= L or JsonSchemaFSM.is_complete(reps[i]):
                continue
            free = _is_free(reps[i])
            if free:
                ensure_chain(i, L - d)
            for c, clo, chi in trie.children(lo, hi, d):
                if free and 0x20 <= c and c != 0x22 and c != 0x5C and trie.last_special_of(clo, chi) <= d:
                    continue  # plain bytes only from here: the chain's rows hold them
                j = int(rows[i][c]) if free else step(i, c)
                if j >= 0:
                    work.append((j, clo, chi, d + 1))
    trans = np.stack(rows) if rows else np.zeros((0, 256), np.int32)
    complete = np.array([JsonSchemaFSM.is_complete(s) for s in reps], dtype=np.uint8)
    return LocalDfa(trans, complete, roots, reps)


# ------------------------------------------------------------------ serving
class JsonSchemaConstraint:
    """Per-sequence JSON-schema constraint over a sampler's mask table.

    Snapshots are interned as table rows (row keys: snapshots that no token
    can tell apart share a row; rows [row0, row0 + n_rows) of the table are
    this constraint's); `rows_for` returns
    the row of each sequence's snapshot and builds the new ones on the
    device in one tgs_mask_rows_from_dfa call; `commit` replays the sampled
    token's bytes (LogitsMasker.commit, ConstrainedGen.swift:827-830)."""

    DFA_CACHE_MAX = 1 << 21  # automaton steps kept across calls before the cache starts over

    def __init__(self, sampler, schema: SchemaNode, tokens, eos: int = -1, row0: int = 0, n_rows: int = 1024,
                 device="cuda:0"):
        from .grammar import token_csr

        self.sampler = sampler
        self.fsm = JsonSchemaFSM(schema)
        self.tokens = [bytes(t) for t in tokens]
        self.eos = int(eos)
        self.trie = TokenTrie(self.tokens)
        self.row0, self.n_rows = int(row0), int(n_rows)
        self.device = device
        self.rows = {}  # canonical key -> table row
        self._dfa_cache = {}  # automaton steps kept across calls (local_dfa's cache)
        off, data = token_csr(self.tokens)
        import torch

        self._off = torch.from_numpy(off).to(device)
        self._data = torch.from_numpy(data).to(device)
        self.built = 0  # rows built on the device so far

    def start(self):
        return self.fsm.start

    def reset(self):
        """Forget every interned snapshot (its rows are free for new ones)."""
        self.rows = {}

    def rows_for(self, snaps, stream=None):
        """Table row of each snapshot (int32 numpy [n]); rows not yet built
        are built on the device (stream order)."""
        import torch

        out = np.empty(len(snaps), dtype=np.int32)
        new = []
        for i, s in enumerate(snaps):
            key = row_key(s, self.trie.max_len)
            r = self.rows.get(key)
            if r is None:
                if len(self.rows) >= self.n_rows:
                    raise RuntimeError("mask-table rows of this constraint are used up")
                r = self.row0 + len(self.rows)
                self.rows[key] = r
                new.append((s, r))
            out[i] = r
        if new:
            if len(self._dfa_cache) > self.DFA_CACHE_MAX:  # bounded memory over a long-lived constraint
                self._dfa_cache.clear()
            dfa = local_dfa([s for s, _ in new], self.trie, cache=self._dfa_cache)
            bc, ct = dfa.byte_classes()
            # The uploads are made and allocated on the stream the rows are built
            # on: the build reads them in stream order, and the allocator does
            # not hand their memory out again (when the next call replaces
            # them) before that stream has passed the build.
            on = torch.cuda.stream(torch.cuda.ExternalStream(stream)) if stream is not None \
                else contextlib.nullcontext()
            with on:
                T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(self.device)
                self._keep = (T(bc), T(ct), T(dfa.complete), T(np.array(dfa.roots, np.int32)),
                              T(np.array([r for _, r in new], np.int32)))
                self.sampler.mask_rows_from_dfa(self._keep[0], self._keep[1], self._keep[2], self._off,
                                                self._data, self._keep[3], self._keep[4], eos=self.eos,
                                                stream=stream)
            self.built += len(new)
        return out

    def commit(self, snap, token_id: int):
        """The snapshot after the sampled token, or None when its bytes are
        rejected (never for a token the mask allowed)."""
        if token_id < 0 or token_id >= len(self.tokens):
            return None
        return JsonSchemaFSM.accept_bytes(snap, self.tokens[token_id])
