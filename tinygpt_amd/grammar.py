"""Host compiler from a GBNF grammar to the byte-level DFA that
tgs_mask_rows_from_dfa replays every token through on the device.

Supported: the non-recursive GBNF subset the reference's grammars use
(grammars/pace-tool-tags.gbnf): rules `name ::= expr`, `#` comments,
"literals" (escapes \\n \\r \\t \\\\ \\" \\xHH), [classes] (ranges, ^, escapes),
rule references (expanded in place; recursion is rejected), ( groups ),
alternation |, and the postfixes * + ? {m} {m,} {m,n}.

The DFA has no dead states: a byte sequence walks from a state without
reaching -1 exactly when some continuation completes the grammar (the
prefix is viable, as the reference's FSMs decide per byte in acceptBytes,
ConstrainedGen.swift:805-822, Serve.swift:2074-2101).  `complete[s]` marks
states that accept and have no way on: there only EOS is allowed, as
LogitsMasker.mask(forFSM:) does when fsm.isComplete.
"""
from __future__ import annotations

import re

import numpy as np

__all__ = ["GrammarError", "Dfa", "compile_gbnf", "token_bytes_table", "token_csr", "PACE_TOOL_TAGS"]


class GrammarError(ValueError):
    pass


# ------------------------------------------------------------------ parsing
_TOKEN = re.compile(
    r"""\s+|\#[^\n]*|(?P<def>::=)|(?P<id>[A-Za-z_][A-Za-z0-9_-]*)|(?P<str>"(?:\\.|[^"\\])*")|"""
    r"""(?P<cls>\[(?:\\.|[^\]\\])*\])|(?P<rep>\{\s*\d+\s*(?:,\s*\d*\s*)?\})|(?P<op>[()|*+?])""",
    re.S,
)


def _unescape(body: str) -> list[int]:
    out, i = [], 0
    esc = {"n": 10, "r": 13, "t": 9, "\\": 92, '"': 34, "'": 39, "]": 93, "[": 91, "-": 45, "^": 94}
    while i < len(body):
        c = body[i]
        if c == "\\":
            if i + 1 >= len(body):
                raise GrammarError("dangling escape")
            d = body[i + 1]
            if d == "x":
                out.append(int(body[i + 2:i + 4], 16))
                i += 4
                continue
            if d not in esc:
                raise GrammarError(f"unknown escape \\{d}")
            out.append(esc[d])
            i += 2
            continue
        out.extend(c.encode("utf-8"))
        i += 1
    return out


def _class_bits(body: str) -> int:
    neg = body.startswith("^")
    if neg:
        body = body[1:]
    items, i = [], 0
    while i < len(body):  # keep escapes as single units
        if body[i] == "\\":
            j = i + 4 if body[i + 1] == "x" else i + 2
            items.append(body[i:j])
            i = j
        else:
            items.append(body[i])
            i += 1
    vals = [_unescape(x) for x in items]
    if any(len(v) != 1 for v in vals):
        raise GrammarError("character classes are single bytes (ASCII)")
    bits, k = 0, 0
    while k < len(items):
        lo = vals[k][0]
        if k + 2 < len(items) and items[k + 1] == "-":
            hi = vals[k + 2][0]
            for b in range(lo, hi + 1):
                bits |= 1 << b
            k += 3
        else:
            bits |= 1 << lo
            k += 1
    return ((1 << 256) - 1) & ~bits if neg else bits


def _tokens(text: str):
    pos, out = 0, []
    while pos < len(text):
        m = _TOKEN.match(text, pos)
        if not m:
            raise GrammarError(f"cannot parse at: {text[pos:pos + 30]!r}")
        pos = m.end()
        kind = m.lastgroup
        if kind:
            out.append((kind, m.group(kind)))
    return out


def _parse(text: str) -> dict:
    toks = _tokens(text)
    rules, i = {}, 0

    def at_rule_start(j):
        return j + 1 < len(toks) and toks[j][0] == "id" and toks[j + 1][0] == "def"

    def parse_alt():
        nonlocal i
        seqs = [parse_seq()]
        while i < len(toks) and toks[i] == ("op", "|"):
            i += 1
            seqs.append(parse_seq())
        return seqs[0] if len(seqs) == 1 else ("alt", seqs)

    def parse_seq():
        nonlocal i
        items = []
        while i < len(toks) and not at_rule_start(i) and toks[i] not in (("op", "|"), ("op", ")")):
            kind, val = toks[i]
            if kind == "str":
                node = ("lit", _unescape(val[1:-1]))
            elif kind == "cls":
                node = ("cls", _class_bits(val[1:-1]))
            elif kind == "id":
                node = ("ref", val)
            elif (kind, val) == ("op", "("):
                i += 1
                node = parse_alt()
                if i >= len(toks) or toks[i] != ("op", ")"):
                    raise GrammarError("unbalanced (")
            else:
                raise GrammarError(f"unexpected {val!r}")
            i += 1
            while i < len(toks) and (toks[i][0] == "rep" or toks[i] in (("op", "*"), ("op", "+"), ("op", "?"))):
                kind, val = toks[i]
                if val == "*":
                    node = ("rep", node, 0, None)
                elif val == "+":
                    node = ("rep", node, 1, None)
                elif val == "?":
                    node = ("rep", node, 0, 1)
                else:
                    parts = val[1:-1].split(",")
                    lo = int(parts[0])
                    hi = lo if len(parts) == 1 else (int(parts[1]) if parts[1].strip() else None)
                    if hi is not None and hi < lo:
                        raise GrammarError(f"bad repetition {val}")
                    node = ("rep", node, lo, hi)
                i += 1
            items.append(node)
        return items[0] if len(items) == 1 else ("seq", items)

    while i < len(toks):
        if not at_rule_start(i):
            raise GrammarError(f"expected a rule at token {toks[i]!r}")
        name = toks[i][1]
        i += 2
        rules[name] = parse_alt()
    if "root" not in rules:
        raise GrammarError("no root rule")
    return rules


# ------------------------------------------------------------------ NFA
class _Nfa:
    def __init__(self):
        self.eps: list[list[int]] = []
        self.edges: list[list[tuple[int, int]]] = []  # (byte bits, target)

    def state(self) -> int:
        self.eps.append([])
        self.edges.append([])
        return len(self.eps) - 1

    def build(self, node, rules, stack=()) -> tuple[int, int]:
        kind = node[0]
        if kind == "lit":
            s = self.state()
            cur = s
            for b in node[1]:
                n = self.state()
                self.edges[cur].append((1 << b, n))
                cur = n
            return s, cur
        if kind == "cls":
            s, e = self.state(), self.state()
            self.edges[s].append((node[1], e))
            return s, e
        if kind == "ref":
            name = node[1]
            if name in stack:
                raise GrammarError(f"recursive rule {name} (only regular grammars compile to a DFA)")
            if name not in rules:
                raise GrammarError(f"undefined rule {name}")
            return self.build(rules[name], rules, stack + (name,))
        if kind == "seq":
            s, cur = None, None
            for it in node[1]:
                a, b = self.build(it, rules, stack)
                if s is None:
                    s = a
                else:
                    self.eps[cur].append(a)
                cur = b
            return s, cur
        if kind == "alt":
            s, e = self.state(), self.state()
            for it in node[1]:
                a, b = self.build(it, rules, stack)
                self.eps[s].append(a)
                self.eps[b].append(e)
            return s, e
        if kind == "rep":
            _, sub, lo, hi = node
            s = self.state()
            cur = s
            for _ in range(lo):
                a, b = self.build(sub, rules, stack)
                self.eps[cur].append(a)
                cur = b
            e = self.state()
            if hi is None:
                a, b = self.build(sub, rules, stack)
                self.eps[cur].append(a)
                self.eps[b].append(a)
                self.eps[b].append(e)
                self.eps[cur].append(e)
            else:
                for _ in range(hi - lo):
                    a, b = self.build(sub, rules, stack)
                    self.eps[cur].append(a)
                    self.eps[cur].append(e)
                    cur = b
                self.eps[cur].append(e)
            return s, e
        raise GrammarError(f"bad node {kind}")


# ------------------------------------------------------------------ DFA
class Dfa:
    """trans: int32 [n, 256] next state (-1: the byte is rejected); accept,
    complete: bool [n]; start state 0."""

    def __init__(self, trans: np.ndarray, accept: np.ndarray):
        self.trans = np.ascontiguousarray(trans, dtype=np.int32)
        self.accept = np.asarray(accept, dtype=bool)
        self.complete = self.accept & (self.trans.max(axis=1) < 0)

    @property
    def n(self) -> int:
        return self.trans.shape[0]

    def byte_classes(self) -> tuple[np.ndarray, np.ndarray]:
        """(byte_class uint8 [256], trans int32 [n, n_cls]): bytes whose
        columns agree in every state share a class, numbered by first byte;
        trans[s, byte_class[b]] == self.trans[s, b]."""
        _, first, inv = np.unique(self.trans.T, axis=0, return_index=True, return_inverse=True)
        order = np.argsort(first)  # class ids in order of their first byte
        rank = np.empty_like(order)
        rank[order] = np.arange(len(order))
        byte_class = rank[inv.reshape(-1)].astype(np.uint8)
        ctrans = np.ascontiguousarray(self.trans[:, np.sort(first)], dtype=np.int32)
        return byte_class, ctrans

    def walk(self, state: int, data: bytes) -> int:
        """State after data from state, or -1 when a byte is rejected."""
        s = state
        for b in data:
            s = int(self.trans[s, b])
            if s < 0:
                return -1
        return s


def _byte_classes(nfa: _Nfa) -> list[int]:
    """Partition of the 256 bytes into classes that every edge set holds
    wholly or not at all; returns class id per byte."""
    sig = [0] * 256
    seen = {}
    k = 0
    for edges in nfa.edges:
        for bits, _ in edges:
            if bits not in seen:
                seen[bits] = k
                k += 1
    cls_of = {}
    out = []
    for b in range(256):
        key = tuple(sorted(v for bits, v in seen.items() if (bits >> b) & 1))
        out.append(cls_of.setdefault(key, len(cls_of)))
    return out


def compile_gbnf(text: str, max_states: int = 200000) -> Dfa:
    rules = _parse(text)
    nfa = _Nfa()
    start, final = nfa.build(("ref", "root"), rules)
    cls = _byte_classes(nfa)
    ncls = max(cls) + 1
    rep = [cls.index(c) for c in range(ncls)]  # one byte per class

    def closure(states) -> frozenset:
        out, todo = set(states), list(states)
        while todo:
            s = todo.pop()
            for t in nfa.eps[s]:
                if t not in out:
                    out.add(t)
                    todo.append(t)
        return frozenset(out)

    d0 = closure([start])
    index = {d0: 0}
    order = [d0]
    trans = []
    qi = 0
    while qi < len(order):
        cur = order[qi]
        qi += 1
        row = [-1] * ncls
        for c in range(ncls):
            b = rep[c]
            nxt = set()
            for s in cur:
                for bits, t in nfa.edges[s]:
                    if (bits >> b) & 1:
                        nxt.add(t)
            if not nxt:
                continue
            cl = closure(nxt)
            if cl not in index:
                if len(order) >= max_states:
                    raise GrammarError(f"DFA beyond {max_states} states")
                index[cl] = len(order)
                order.append(cl)
            row[c] = index[cl]
        trans.append(row)
    accept = np.array([final in st for st in order], dtype=bool)
    tc = np.array(trans, dtype=np.int64)
    # drop states from which no accepting state can be reached
    live = accept.copy()
    changed = True
    while changed:
        reach = np.zeros_like(live)
        ok = tc >= 0
        reach |= (ok & live[np.where(ok, tc, 0)]).any(axis=1)
        new = live | reach
        changed = bool((new != live).any())
        live = new
    if not live[0]:
        raise GrammarError("the grammar accepts nothing")
    remap = -np.ones(len(order), dtype=np.int64)
    remap[live] = np.arange(int(live.sum()))
    tc = np.where(tc >= 0, remap[np.where(tc >= 0, tc, 0)], -1)[live]
    full = tc[:, np.array(cls)]  # [n, 256]
    return Dfa(full.astype(np.int32), accept[live])


def token_bytes_table(vocab_size: int, decode=None) -> list[bytes]:
    """The per-id byte strings that grammar masks test, built as the server
    builds them at start-up (native-mac/Sources/TinyGPTServe/Serve.swift:398-408,
    `Array(tok.decode([id]).utf8)` for every id): each id decoded on its own
    and the string encoded as UTF-8.

    decode None: the byte-level tokenizer of the from-scratch models
      (TokenizerBox.byteLevel, Serve.swift:1887-1893; ByteTokenizer.decode,
      native-mac/Sources/TinyGPTModel/Tokenizer.swift:35-41): an id below 256
      is that byte, decoded as UTF-8 with each invalid sequence replaced by
      U+FFFD.  Ids 0-127 give their byte; ids 128-255 (a lone non-ASCII byte)
      give EF BF BD; ids from 256 on give no bytes.
    decode a callable (list of ids -> str): an HF tokenizer's decode
      (HFTokenizer.decode calls swift-transformers' decode(tokens:), which
      keeps special tokens), e.g. `lambda ids: tok.decode(ids,
      skip_special_tokens=False)` for a `tokenizers.Tokenizer`.  A token
      holding part of a multi-byte character decodes to U+FFFD there too, so
      its entry is EF BF BD, not its own bytes.
    """
    if decode is None:
        return [bytes([i]).decode("utf-8", errors="replace").encode("utf-8") if i < 256 else b""
                for i in range(vocab_size)]
    return [decode([i]).encode("utf-8") for i in range(vocab_size)]


def token_csr(tokens: list[bytes]) -> tuple[np.ndarray, np.ndarray]:
    """Token byte strings as (offsets int32 [V + 1], bytes uint8) for
    tgs_mask_rows_from_dfa."""
    lens = np.array([len(t) for t in tokens], dtype=np.int64)
    off = np.zeros(len(tokens) + 1, dtype=np.int64)
    np.cumsum(lens, out=off[1:])
    if off[-1] >= 2**31:
        raise ValueError("token bytes beyond 2 GiB")
    data = np.frombuffer(b"".join(tokens), dtype=np.uint8).copy() if off[-1] else np.zeros(1, np.uint8)
    return off.astype(np.int32), data


# The byte language PaceToolTagFSM accepts (Serve.swift:2058-2182): free text
# of printable ASCII without brackets, then one tag; nothing after its "]".
# (grammars/pace-tool-tags.gbnf is the offline form of the same constraint;
# its counted `sentence` repetition over a class holding the separator has no
# small DFA, and the server masks with the FSM above, not with that file.)
PACE_TOOL_TAGS = r'''
root   ::= text "[" tag
text   ::= [\x20-\x5a\x5c\x5e-\x7e]*
tag    ::= "POINT:none]" | "POINT:" coords ":" label "]" | "CLICK:" coords ":" label "]"
         | "TYPE:" [A-Za-z0-9 _.,!?'"\-]{1,200} "]"
         | "SCROLL:" ("up" | "down" | "left" | "right") ":" [0-9]{1,4} "]"
         | "KEY:" [A-Za-z+]{1,30} "]"
         | "OPEN_APP:" [A-Za-z] [A-Za-z0-9 ]{0,30} "]"
coords ::= [0-9]{1,4} "," [0-9]{1,4}
label  ::= [A-Za-z] [A-Za-z0-9 _\-]{0,40}
'''
