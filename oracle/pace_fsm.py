"""Restatement of the reference server's tool-tag FSM and token masker, for
tests only (TEST INFRASTRUCTURE: imported by tests/ and bench.py's
cpu_baseline leg as the checker, never by the product).

PaceToolTagFSM (native-mac/Sources/TinyGPTServe/Serve.swift:2058-2182):
a byte history is viable when it decodes as UTF-8, the text before the
first "[" is printable ASCII without brackets (:2103-2107) and the rest is a
prefix of one tag form (:2109-2139, coordsLabelPrefix :2141-2154,
scrollPrefix :2156-2165, bodyPrefix :2173-2190); complete when that rest is a
whole tag (isCompleteTag :2203-2206).  ServeTokenMasker.mask(for:)
(:2005-2025): a complete FSM allows no token; otherwise a non-empty token is
allowed when every one of its bytes keeps the history viable."""
from __future__ import annotations

import re

_COMPLETE = re.compile(
    r"^\[(POINT:none|POINT:[0-9]{1,4},[0-9]{1,4}:[A-Za-z][A-Za-z0-9 _-]{0,40}|"
    r"CLICK:[0-9]{1,4},[0-9]{1,4}:[A-Za-z][A-Za-z0-9 _-]{0,40}|TYPE:[A-Za-z0-9 _.,!?'\"-]{1,200}|"
    r"SCROLL:(up|down|left|right):[0-9]{1,4}|KEY:[A-Za-z+]{1,30}|OPEN_APP:[A-Za-z][A-Za-z0-9 ]{0,30})\]$"
)


def _digit(c):
    return "0" <= c <= "9"


def _alpha(c):
    return ("A" <= c <= "Z") or ("a" <= c <= "z")


def _key(c):
    return _alpha(c) or c == "+"


def _app(c):
    return _alpha(c) or _digit(c) or c == " "


def _label(c):
    return _alpha(c) or _digit(c) or c in " _-"


def _type(c):
    return _alpha(c) or _digit(c) or c in " _-.,!?'\""


def _text(c):
    v = ord(c)
    if v in (0x0A, 0x0D, 0x09) or c in "[]":
        return False
    return 0x20 <= v <= 0x7E


def _body_prefix(s, lo, hi, first, rest):
    if not s:
        return True
    count = 0
    for idx, c in enumerate(s):
        if c == "]":
            return idx == len(s) - 1 and count >= lo
        ok = first(c) if count == 0 else rest(c)
        if not ok:
            return False
        count += 1
        if count > hi:
            return False
    return True


def _consume_digits(s, i, hi):
    count = 0
    while i < len(s) and _digit(s[i]):
        count += 1
        if count > hi:
            return count, i
        i += 1
    return count, i


def _coords_label_prefix(s):
    x, i = _consume_digits(s, 0, 4)
    if i == len(s):
        return x <= 4
    if not (x >= 1 and s[i] == ","):
        return False
    i += 1
    y, i = _consume_digits(s, i, 4)
    if i == len(s):
        return y <= 4
    if not (y >= 1 and s[i] == ":"):
        return False
    i += 1
    return _body_prefix(s[i:], 1, 41, _alpha, _label)


def _scroll_prefix(s):
    for d in ("up", "down", "left", "right"):
        if d.startswith(s):
            return True
        if s.startswith(d + ":"):
            return _body_prefix(s[len(d) + 1:], 1, 4, _digit, _digit)
    return False


def _tag_prefix(tag):
    if "[POINT:none]".startswith(tag):
        return True
    if tag.startswith("[POINT:"):
        return _coords_label_prefix(tag[len("[POINT:"):])
    if "[POINT:".startswith(tag):
        return True
    if tag.startswith("[CLICK:"):
        return _coords_label_prefix(tag[len("[CLICK:"):])
    if "[CLICK:".startswith(tag):
        return True
    if tag.startswith("[TYPE:"):
        return _body_prefix(tag[len("[TYPE:"):], 1, 200, _type, _type)
    if "[TYPE:".startswith(tag):
        return True
    if tag.startswith("[SCROLL:"):
        return _scroll_prefix(tag[len("[SCROLL:"):])
    if "[SCROLL:".startswith(tag):
        return True
    if tag.startswith("[KEY:"):
        return _body_prefix(tag[len("[KEY:"):], 1, 30, _key, _key)
    if "[KEY:".startswith(tag):
        return True
    if tag.startswith("[OPEN_APP:"):
        return _body_prefix(tag[len("[OPEN_APP:"):], 1, 31, _alpha, _app)
    if "[OPEN_APP:".startswith(tag):
        return True
    return False


def is_viable(data: bytes) -> bool:
    try:
        text = data.decode("utf-8")
    except UnicodeDecodeError:
        return False
    b = text.find("[")
    if b < 0:
        return all(_text(c) for c in text)
    if not all(_text(c) for c in text[:b]):
        return False
    return _tag_prefix(text[b:])


def is_complete(data: bytes) -> bool:
    try:
        text = data.decode("utf-8")
    except UnicodeDecodeError:
        return False
    b = text.find("[")
    return b >= 0 and _COMPLETE.match(text[b:]) is not None


def accept_bytes(history: bytes, new: bytes) -> bool:
    """PaceToolTagFSM.acceptBytes (:2074-2082): every prefix stays viable."""
    cand = bytearray(history)
    for x in new:
        cand.append(x)
        if not is_viable(bytes(cand)):
            return False
    return True


def mask(history: bytes, tokens: list[bytes]) -> list[bool]:
    """ServeTokenMasker.mask(for:) (:2005-2025) as allowed flags."""
    if is_complete(history):
        return [False] * len(tokens)
    return [bool(t) and accept_bytes(history, t) for t in tokens]
