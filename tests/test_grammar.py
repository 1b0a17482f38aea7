"""The host grammar compiler (tinygpt_amd.grammar) and the DFA replay
oracle, pinned against independent checkers.  CPU only.

- The tool-tag DFA against a restatement of the reference server's FSM
  (oracle/pace_fsm.py, Serve.swift:2058-2182) on generated strings: viable
  prefixes and complete tags agree.
- The GBNF compiler against the `regex` module's partial matching on small
  grammars: a string walks without rejection exactly when some extension
  matches, and ends in an accepting state exactly when it matches.
- The vectorised mask-row oracle against the FSM's per-token replay
  (ServeTokenMasker.mask(for:), Serve.swift:2005-2025)."""
import numpy as np
import pytest

from tinygpt_amd import grammar as G

TAG_FORMS = ["POINT:none", "POINT:{d},{d}:{l}", "CLICK:{d},{d}:{l}", "TYPE:{t}", "SCROLL:{s}:{d}", "KEY:{k}",
             "OPEN_APP:{a}"]


def _gen_strings(g, n):
    out = []
    alpha = "abcXYZ"
    for _ in range(n):
        text = "".join(g.choice(list("hello wor,ld.!?'0123")) for _ in range(g.integers(0, 8)))
        form = TAG_FORMS[g.integers(len(TAG_FORMS))]
        d = lambda: "".join(g.choice(list("0123456789")) for _ in range(g.integers(0, 6)))
        body = (form.replace("{d}", d(), 1).replace("{d}", d(), 1)
                .replace("{l}", "".join(g.choice(list(alpha + " _-9")) for _ in range(g.integers(0, 45))))
                .replace("{t}", "".join(g.choice(list(alpha + " .,'\"-")) for _ in range(g.integers(0, 205))))
                .replace("{s}", g.choice(["up", "down", "left", "right", "u", "dow", "x"]))
                .replace("{k}", "".join(g.choice(list(alpha + "+")) for _ in range(g.integers(0, 33))))
                .replace("{a}", "".join(g.choice(list(alpha + " 7")) for _ in range(g.integers(0, 34)))))
        s = (text + "[" + body + ("]" if g.random() < 0.7 else "")).encode()
        cut = int(g.integers(0, len(s) + 1)) if g.random() < 0.5 else len(s)
        s = s[:cut]
        if g.random() < 0.3:
            s += bytes([int(g.integers(0, 256))])
        out.append(s)
    return out


def test_tool_tag_dfa_matches_the_reference_fsm(oracle):
    import pace_fsm as P

    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    g = np.random.default_rng(5)
    strings = _gen_strings(g, 6000) + [b"", b"[", b"x]", b"a[POINT:none]", b"a[POINT:none]b", b"\xc3\xa9"]
    n_viable = n_complete = 0
    for s in strings:
        st = d.walk(0, s)
        assert (st >= 0) == P.is_viable(s), s
        if st >= 0:
            assert bool(d.accept[st]) == P.is_complete(s), s
            assert bool(d.complete[st]) == P.is_complete(s), s
            n_viable += 1
            n_complete += bool(d.accept[st])
    assert n_viable > 1000 and n_complete > 300  # both sides of each check exercised


@pytest.mark.parametrize("gbnf,pattern", [
    (r'''root ::= "ab" [0-9]{1,3} ("x" | "yz")*''', r"ab[0-9]{1,3}(?:x|yz)*"),
    (r'''root ::= item ("," item){0,2} "."
         item ::= [^,.\x00-\x1f]+ | "\"" [a-c]? "\""''', r'(?:[^,.\x00-\x1f]+|"[a-c]?")(?:,(?:[^,.\x00-\x1f]+|"[a-c]?")){0,2}\.'),
    (r'''root ::= ("a" "b"?)+ [xy]{2,} # comment
         ''', r"(?:ab?)+[xy]{2,}"),
])
def test_gbnf_compiler_against_regex_partial_matching(gbnf, pattern):
    import regex

    d = G.compile_gbnf(gbnf)
    rx = regex.compile(pattern.encode("latin-1"))
    g = np.random.default_rng(7)
    alphabet = list(b'abxyz012,."c\x01 ')
    for _ in range(4000):
        s = bytes(int(g.choice(alphabet)) for _ in range(g.integers(0, 9)))
        st = d.walk(0, s)
        viable = rx.fullmatch(s, partial=True) is not None
        assert (st >= 0) == viable, s
        if st >= 0:
            assert bool(d.accept[st]) == (rx.fullmatch(s) is not None), s


def test_gbnf_errors():
    with pytest.raises(G.GrammarError):
        G.compile_gbnf('root ::= a\na ::= "x" a')  # recursion
    with pytest.raises(G.GrammarError):
        G.compile_gbnf('start ::= "x"')  # no root
    with pytest.raises(G.GrammarError):
        G.compile_gbnf('root ::= "x" undefined')


def test_mask_row_oracle_matches_per_token_replay(oracle):
    import pace_fsm as P

    d = G.compile_gbnf(G.PACE_TOOL_TAGS)
    g = np.random.default_rng(9)
    pieces = [b"[", b"]", b"POINT", b":", b"none", b",", b"CLICK", b"TYPE", b"SCROLL", b"up", b"KEY", b"+",
              b"OPEN_APP", b" ", b"_", b"-", b"\n", b"\xc3", b"\xa9", b"hello", b"12", b"9", b"x"]
    tokens = [b""] + [b"".join(g.choice(pieces) for _ in range(g.integers(1, 4))) for _ in range(700)]
    histories = [b"", b"ok ", b"ok [", b"ok [POINT:", b"ok [POINT:1", b"ok [POINT:12,3:Sa", b"[TYPE:abc",
                 b"[SCROLL:up:", b"[KEY:cmd", b"[POINT:none]", b"[OPEN_APP:Sa 1"]
    states = [d.walk(0, h) for h in histories]
    assert min(states) >= 0
    rows = oracle.dfa_mask_rows(d.trans, d.complete, tokens, states)
    for h, row in zip(histories, rows):
        want = P.mask(h, tokens)
        got = [(int(row[v >> 5]) >> (v & 31)) & 1 == 1 for v in range(len(tokens))]
        assert got == want, h
