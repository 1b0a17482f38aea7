"""TEST INFRASTRUCTURE ONLY (imported by tests/ alone): a second, direct
restatement of the reference's JSON-schema automaton and masker, written
as the reference is (a mutable frame stack, clone per token), to check the
product's immutable automaton, its canonical state keys and its device
DFA rows against.

  JSONSchemaNode.parse   native-mac/Sources/TinyGPTModel/JSONSchema.swift:72-116
  JSONSchemaFSM          native-mac/Sources/TinyGPTModel/ConstrainedGen.swift:35-749
  LogitsMasker           native-mac/Sources/TinyGPTModel/ConstrainedGen.swift:775-837

Schema nodes are plain dicts: {"t": "object", "props": [(key, node)],
"req": set}, {"t": "string", "enum": list|None, "min": int|None, "max":
int|None}, {"t": "number", "int": bool}, {"t": "boolean"}, {"t": "null"},
{"t": "array", "items": node}, {"t": "any"}.
"""
from __future__ import annotations

import json


def _as_int(v):
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    if isinstance(v, float) and v != int(v):
        return None
    return int(v)


def parse(any_):
    """JSONSchema.swift:72-116."""
    if not isinstance(any_, dict):
        return {"t": "any"}
    enum_arr = any_.get("enum")
    if isinstance(enum_arr, list):
        strings = [x for x in enum_arr if isinstance(x, str)]
        if len(strings) > 0:
            return {"t": "string", "enum": strings, "min": _as_int(any_.get("minLength")),
                    "max": _as_int(any_.get("maxLength"))}
    typ = any_.get("type")
    if not isinstance(typ, str):
        return {"t": "any"}
    if typ == "object":
        props_raw = any_.get("properties") if isinstance(any_.get("properties"), dict) else {}
        props = [(k, parse(props_raw[k])) for k in sorted(props_raw.keys())]
        r = any_.get("required")
        req = set(r) if isinstance(r, list) and all(isinstance(x, str) for x in r) else set()
        return {"t": "object", "props": props, "req": req}
    if typ == "string":
        return {"t": "string", "enum": None, "min": _as_int(any_.get("minLength")), "max": _as_int(any_.get("maxLength"))}
    if typ == "number":
        return {"t": "number", "int": False}
    if typ == "integer":
        return {"t": "number", "int": True}
    if typ == "boolean":
        return {"t": "boolean"}
    if typ == "null":
        return {"t": "null"}
    if typ == "array":
        return {"t": "array", "items": parse(any_.get("items"))}
    return {"t": "any"}


def from_json(text):
    return parse(json.loads(text))


ANY = {"t": "any"}
EMPTY_OBJECT = {"t": "object", "props": [], "req": set()}


class FSM:
    """JSONSchemaFSM.  Frames are dicts with a "k" kind field; a transition
    builds a new frame and never edits one in place, so a copy of the stack
    list is a full copy of the state (Swift's value-type frames)."""

    def __init__(self, root):
        self.stack = [{"k": "value", "schema": root, "phase": "start"}]
        self.last_popped_key = None

    def clone(self):
        c = FSM(ANY)
        c.stack = list(self.stack)
        c.last_popped_key = self.last_popped_key
        return c

    @property
    def is_complete(self):
        return len(self.stack) == 1 and self.stack[0]["k"] == "value" and self.stack[0]["phase"] == "done"

    def accept_byte(self, b):
        return self._drive(b, 0)

    def accept_bytes(self, data):
        snap = list(self.stack)
        snap_key = self.last_popped_key
        for b in data:
            if not self._drive(b, 0):
                self.stack = snap
                self.last_popped_key = snap_key
                return False
        return True

    def accept_string(self, s):
        return self.accept_bytes(s.encode("utf-8"))

    # ---- driver (ConstrainedGen.swift:217-266)
    def _drive(self, b, depth):
        if depth > 64:
            return False
        if b in (0x20, 0x09, 0x0A, 0x0D) and self._allows_ws():
            return True
        if not self.stack:
            return False
        top = self.stack[-1]
        act = self._transition(top, b)
        kind = act[0]
        if kind == "reject":
            return False
        if kind == "replace":
            self.stack[-1] = act[1]
            return True
        if kind == "push":
            self.stack.append(act[1])
            return True
        if kind == "replaceAndPush":
            self.stack[-1] = act[1]
            self.stack.append(act[2])
            return True
        if kind == "pushAndRetry":
            self.stack.append(act[1])
            ok = self._drive(b, depth + 1)
            if not ok:
                self.stack.pop()
            return ok
        if kind == "popConsuming":
            if top["k"] == "string" and top["isKey"]:
                self.last_popped_key = top["content"]
            self.stack.pop()
            self._advance_parent()
            return True
        if kind == "popAndRetry":
            self.stack.pop()
            self._advance_parent()
            return self._drive(b, depth + 1)
        raise AssertionError(kind)

    def _allows_ws(self):
        return False  # minified JSON only (ConstrainedGen.swift:285-297)

    def _advance_parent(self):
        while self.stack:
            parent = self.stack[-1]
            if parent["k"] == "object":
                of = dict(parent)
                if of["phase"] in ("afterOpen", "afterComma"):
                    key = self.last_popped_key if self.last_popped_key is not None else ""
                    self.last_popped_key = None
                    of["phase"] = "afterKey"
                    of["key"] = key
                elif of["phase"] == "insideValue":
                    of["emitted"] = set(of["emitted"]) | {of["key"]}
                    of["phase"] = "afterValue"
                self.stack[-1] = of
                return
            if parent["k"] == "array":
                af = dict(parent)
                af["phase"] = "afterItem"
                self.stack[-1] = af
                return
            if parent["k"] == "value":
                if len(self.stack) == 1:
                    self.stack[-1] = {"k": "value", "schema": parent["schema"], "phase": "done"}
                    return
                self.stack.pop()
                continue
            return

    # ---- transitions
    def _transition(self, top, b):
        k = top["k"]
        if k == "value":
            if top["phase"] == "done":
                return ("reject",)
            return self._open_value(top["schema"], b)
        if k == "object":
            return self._step_object(top, b)
        if k == "array":
            return self._step_array(top, b)
        if k == "string":
            return self._step_string(top, b)
        if k == "number":
            return self._step_number(top, b)
        if k == "boolean":
            return self._step_boolean(top, b)
        if k == "null":
            return self._step_null(top, b)
        raise AssertionError(k)

    @staticmethod
    def _string(enum, mn, mx, is_key):
        return {"k": "string", "state": "body", "digits": 0, "enum": enum, "min": mn, "max": mx, "content": "",
                "isKey": is_key}

    def _open_value(self, schema, b):
        t = schema["t"]
        if t == "any":
            return self._open_any(b)
        if t == "object":
            if b != ord("{"):
                return ("reject",)
            return ("push", {"k": "object", "schema": schema, "emitted": set(), "phase": "afterOpen", "key": None})
        if t == "array":
            if b != ord("["):
                return ("reject",)
            return ("push", {"k": "array", "items": schema["items"], "phase": "afterOpen"})
        if t == "string":
            if b != ord('"'):
                return ("reject",)
            return ("push", self._string(schema["enum"], schema["min"], schema["max"], False))
        if t == "number":
            if b == ord("-"):
                return ("push", {"k": "number", "state": "sign", "int": schema["int"]})
            if 0x30 <= b <= 0x39:
                return ("push", {"k": "number", "state": "intZero" if b == 0x30 else "intDigits", "int": schema["int"]})
            return ("reject",)
        if t == "boolean":
            if b == ord("t"):
                return ("push", {"k": "boolean", "lit": "true", "pos": 1})
            if b == ord("f"):
                return ("push", {"k": "boolean", "lit": "false", "pos": 1})
            return ("reject",)
        if t == "null":
            if b == ord("n"):
                return ("push", {"k": "null", "pos": 1})
            return ("reject",)
        raise AssertionError(t)

    def _open_any(self, b):
        c = chr(b)
        if c == "{":
            return ("push", {"k": "object", "schema": EMPTY_OBJECT, "emitted": set(), "phase": "afterOpen", "key": None})
        if c == "[":
            return ("push", {"k": "array", "items": ANY, "phase": "afterOpen"})
        if c == '"':
            return ("push", self._string(None, None, None, False))
        if c == "-":
            return ("push", {"k": "number", "state": "sign", "int": False})
        if c == "t":
            return ("push", {"k": "boolean", "lit": "true", "pos": 1})
        if c == "f":
            return ("push", {"k": "boolean", "lit": "false", "pos": 1})
        if c == "n":
            return ("push", {"k": "null", "pos": 1})
        if 0x30 <= b <= 0x39:
            return ("push", {"k": "number", "state": "intZero" if b == 0x30 else "intDigits", "int": False})
        return ("reject",)

    @staticmethod
    def _unemitted(schema, emitted):
        if schema["t"] == "object":
            if not schema["props"]:
                return None
            return [k for k, _ in schema["props"] if k not in emitted]
        return None

    @staticmethod
    def _schema_for(key, schema):
        if schema["t"] == "object":
            for k, v in schema["props"]:
                if k == key:
                    return v
        return ANY

    def _step_object(self, of, b):
        ph = of["phase"]
        if ph == "afterOpen":
            if b == ord("}"):
                if of["schema"]["t"] == "object" and not of["schema"]["req"] <= of["emitted"]:
                    return ("reject",)
                return ("popConsuming",)
            if b == ord('"'):
                keys = self._unemitted(of["schema"], of["emitted"])
                if keys is not None and len(keys) == 0:
                    return ("reject",)
                return ("push", self._string(keys, None, None, True))
            return ("reject",)
        if ph == "afterComma":
            if b == ord('"'):
                keys = self._unemitted(of["schema"], of["emitted"])
                if keys is not None and len(keys) == 0:
                    return ("reject",)
                return ("push", self._string(keys, None, None, True))
            return ("reject",)
        if ph == "afterKey":
            if b == ord(":"):
                nf = dict(of)
                nf["phase"] = "insideValue"
                return ("replaceAndPush", nf, {"k": "value", "schema": self._schema_for(of["key"], of["schema"]),
                                               "phase": "start"})
            return ("reject",)
        if ph == "insideValue":
            return ("reject",)
        if ph == "afterValue":
            if b == ord(","):
                rem = self._unemitted(of["schema"], of["emitted"])
                if rem is not None and len(rem) == 0:
                    return ("reject",)
                nf = dict(of)
                nf["phase"] = "afterComma"
                return ("replace", nf)
            if b == ord("}"):
                if of["schema"]["t"] == "object" and not of["schema"]["req"] <= of["emitted"]:
                    return ("reject",)
                return ("popConsuming",)
            return ("reject",)
        return ("reject",)

    def _step_array(self, af, b):
        ph = af["phase"]
        if ph == "afterOpen":
            if b == ord("]"):
                return ("popConsuming",)
            return ("pushAndRetry", {"k": "value", "schema": af["items"], "phase": "start"})
        if ph == "afterComma":
            return ("pushAndRetry", {"k": "value", "schema": af["items"], "phase": "start"})
        if ph == "afterItem":
            if b == ord(","):
                nf = dict(af)
                nf["phase"] = "afterComma"
                return ("replace", nf)
            if b == ord("]"):
                return ("popConsuming",)
            return ("reject",)
        return ("reject",)

    def _step_string(self, sf, b):
        st = sf["state"]
        if st == "body":
            if b == ord('"'):
                if sf["enum"] is not None and sf["content"] not in sf["enum"]:
                    return ("reject",)
                if sf["min"] is not None and len(sf["content"]) < sf["min"]:
                    return ("reject",)
                return ("popConsuming",)
            if b == ord("\\"):
                if sf["enum"] is not None:
                    return ("reject",)
                nf = dict(sf)
                nf["state"] = "escape"
                return ("replace", nf)
            if b < 0x20:
                return ("reject",)
            new_prefix = sf["content"] + chr(b)  # String(UnicodeScalar(b))
            if sf["max"] is not None and len(new_prefix) > sf["max"]:
                return ("reject",)
            if sf["enum"] is not None and not any(v.startswith(new_prefix) for v in sf["enum"]):
                return ("reject",)
            nf = dict(sf)
            nf["content"] = new_prefix
            return ("replace", nf)
        if st == "escape":
            if chr(b) in '"\\/bfnrt':
                nf = dict(sf)
                nf["state"] = "body"
                nf["content"] = sf["content"] + "\\" + chr(b)
                if sf["max"] is not None and len(nf["content"]) > sf["max"]:
                    return ("reject",)
                return ("replace", nf)
            if b == ord("u"):
                nf = dict(sf)
                nf["state"] = "unicode"
                nf["digits"] = 0
                nf["content"] = sf["content"] + "\\u"
                if sf["max"] is not None and len(nf["content"]) > sf["max"]:
                    return ("reject",)
                return ("replace", nf)
            return ("reject",)
        if st == "unicode":
            if chr(b) in "0123456789abcdefABCDEF":
                nf = dict(sf)
                nf["content"] = sf["content"] + chr(b)
                if sf["max"] is not None and len(nf["content"]) > sf["max"]:
                    return ("reject",)
                if sf["digits"] + 1 == 4:
                    nf["state"] = "body"
                    nf["digits"] = 0
                else:
                    nf["digits"] = sf["digits"] + 1
                return ("replace", nf)
            return ("reject",)
        return ("reject",)

    def _step_number(self, nf, b):
        term = b in (ord(","), ord("}"), ord("]"), 0x20, 0x09, 0x0A, 0x0D)
        st = nf["state"]
        if term:
            return ("popAndRetry",) if st in ("intZero", "intDigits", "fracDigits", "expDigits") else ("reject",)
        digit = 0x30 <= b <= 0x39

        def to(s):
            x = dict(nf)
            x["state"] = s
            return ("replace", x)

        if st == "sign":
            if b == 0x30:
                return to("intZero")
            return to("intDigits") if digit else ("reject",)
        if st == "intZero":
            if b == ord(".") and not nf["int"]:
                return to("afterFracPoint")
            if b in (ord("e"), ord("E")) and not nf["int"]:
                return to("afterExp")
            return ("reject",)
        if st == "intDigits":
            if digit:
                return ("replace", nf)
            if b == ord(".") and not nf["int"]:
                return to("afterFracPoint")
            if b in (ord("e"), ord("E")) and not nf["int"]:
                return to("afterExp")
            return ("reject",)
        if st == "afterFracPoint":
            return to("fracDigits") if digit else ("reject",)
        if st == "fracDigits":
            if digit:
                return ("replace", nf)
            if b in (ord("e"), ord("E")):
                return to("afterExp")
            return ("reject",)
        if st == "afterExp":
            if b in (ord("+"), ord("-")):
                return to("expSign")
            return to("expDigits") if digit else ("reject",)
        if st == "expSign":
            return to("expDigits") if digit else ("reject",)
        if st == "expDigits":
            return ("replace", nf) if digit else ("reject",)
        return ("reject",)

    @staticmethod
    def _step_boolean(f, b):
        chars = f["lit"].encode()
        pos = f["pos"]
        if pos >= len(chars):
            return ("reject",)
        if b == chars[pos]:
            if pos + 1 == len(chars):
                return ("popConsuming",)
            return ("replace", {"k": "boolean", "lit": f["lit"], "pos": pos + 1})
        return ("reject",)

    @staticmethod
    def _step_null(f, b):
        chars = b"null"
        pos = f["pos"]
        if pos >= len(chars):
            return ("reject",)
        if b == chars[pos]:
            if pos + 1 == len(chars):
                return ("popConsuming",)
            return ("replace", {"k": "null", "pos": pos + 1})
        return ("reject",)


def masker_row(fsm: FSM, token_bytes, eos=None):
    """LogitsMasker.mask(forFSM:) (ConstrainedGen.swift:805-822) as a bool
    row: True where the reference's mask is 0."""
    out = [False] * len(token_bytes)
    if fsm.is_complete:
        if eos is not None and 0 <= eos < len(out):
            out[eos] = True
        return out
    for i, t in enumerate(token_bytes):
        if len(t) == 0:
            continue
        probe = fsm.clone()
        if probe.accept_bytes(t):
            out[i] = True
    return out
