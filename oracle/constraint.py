"""TEST INFRASTRUCTURE ONLY — pure-Python restatement of the reference's decode-based
constraint (crates/bfi-runtime/src/sample.rs:63-291), the checker of the allow-mask producer.

Strings are handled as UTF-8 bytes, as the reference's `str` methods compare them. Each
function cites the reference lines it follows. Only tests/ import this module.

Pinned by: the reference's constraint tests (sample.rs:505-581, restated as known answers in
tests/test_oracle_constraint.py); for json_object_prefix_ok, Python's json module on complete
objects and on every prefix of them, and brute force over all strings of up to six structural
characters against an independent statement of the scan (strings collapsed by a regular
expression, the depth as a running sum); for json_name_so_far and tool_call_prefix_ok,
hand-derived cases (the key's restart after a non-colon, escapes, prefixes of several names)
and brute force over more than 100,000 short strings of the bytes that decide the scan
against an independent statement (a regular-expression search); for the grammar parsers,
hand-derived cases and Rust's White_Space set, with and without whitespace on either side.
"""
from __future__ import annotations

# Rust's char::is_whitespace (Unicode White_Space), used by str::trim in strip_root /
# parse_id_union (sample.rs:208-234).
_RUST_WS = set(
    [0x09, 0x0A, 0x0B, 0x0C, 0x0D, 0x20, 0x85, 0xA0, 0x1680, 0x2028, 0x2029, 0x202F, 0x205F, 0x3000]
    + list(range(0x2000, 0x200B))
)

# u8::is_ascii_whitespace: space, \t, \n, form feed, \r (not \v) — sample.rs:144-206, 236-286.
_ASCII_WS = {0x20, 0x09, 0x0A, 0x0C, 0x0D}

TOOL_NONE, TOOL_AUTO, TOOL_REQUIRED, TOOL_NAMED = 0, 1, 2, 3


def rust_trim(s: str) -> str:
    a, b = 0, len(s)
    while a < b and ord(s[a]) in _RUST_WS:
        a += 1
    while b > a and ord(s[b - 1]) in _RUST_WS:
        b -= 1
    return s[a:b]


def strip_root(g: str):
    """sample.rs:230-234."""
    s = rust_trim(g)
    if not s.startswith("root"):
        return None
    rest = rust_trim(s[4:])
    if not rest.startswith("::="):
        return None
    return rust_trim(rest[3:])


def _parse_u32(t: str):
    # str::parse::<u32>: optional '+', then one or more ASCII digits, no overflow
    if t.startswith("+"):
        t = t[1:]
    if not t or any(c not in "0123456789" for c in t):
        return None
    v = int(t)
    return v if v <= 0xFFFFFFFF else None


def parse_id_union(g: str):
    """sample.rs:208-221: `root ::= id(1) | id(2)` -> set of ids, else None."""
    rest = strip_root(g)
    if rest is None:
        return None
    out = set()
    for part in rest.split("|"):
        p = rust_trim(part)
        if not (p.startswith("id(") and p.endswith(")")) or len(p) < 4:
            return None
        v = _parse_u32(rust_trim(p[3:-1]))
        if v is None:
            return None
        out.add(v)
    return out or None


def parse_literal_root(g: str):
    """sample.rs:222-228: `root ::= "hello"` -> "hello" (up to the next quote)."""
    rest = strip_root(g)
    if rest is None or not rest.startswith('"'):
        return None
    rest = rest[1:]
    end = rest.find('"')
    return None if end < 0 else rest[:end]


def json_object_prefix_ok(b: bytes) -> bool:
    """sample.rs:236-286."""
    i, n = 0, len(b)
    while i < n and b[i] in _ASCII_WS:
        i += 1
    if i == n:
        return True
    if b[i] != ord("{"):
        return False
    depth, in_string, escape = 0, False, False
    while i < n:
        c = b[i]
        if in_string:
            if escape:
                escape = False
            elif c == ord("\\"):
                escape = True
            elif c == ord('"'):
                in_string = False
            i += 1
            continue
        if c == ord('"'):
            in_string = True
        elif c in (ord("{"), ord("[")):
            depth += 1
        elif c in (ord("}"), ord("]")):
            depth -= 1
            if depth < 0:
                return False
            if depth == 0:
                i += 1
                while i < n:
                    if b[i] not in _ASCII_WS:
                        return False
                    i += 1
                return True
        i += 1
    return in_string or escape or depth > 0


def json_name_so_far(b: bytes):
    """sample.rs:144-206: ("missing",), ("partial", bytes), ("complete", bytes), ("invalid",)."""
    i, n = 0, len(b)
    while i + 6 <= n:
        if b[i:i + 6] == b'"name"':
            j = i + 6
            while j < n and b[j] in _ASCII_WS:
                j += 1
            if j >= n:
                return ("missing",)
            if b[j] != ord(":"):
                i += 1
                continue
            j += 1
            while j < n and b[j] in _ASCII_WS:
                j += 1
            if j >= n:
                return ("partial", b"")
            if b[j] != ord('"'):
                return ("invalid",)
            j += 1
            start, escaped, closed = j, False, False
            while j < n:
                c = b[j]
                if escaped:
                    escaped = False
                    j += 1
                    continue
                if c == ord("\\"):
                    escaped = True
                    j += 1
                    continue
                if c == ord('"'):
                    closed = True
                    break
                j += 1
            return ("complete" if closed else "partial", b[start:j])
        i += 1
    return ("missing",)


def tool_call_prefix_ok(b: bytes, choice: int, named: bytes, names) -> bool:
    """sample.rs:110-136 (choice: TOOL_* above; `named` the Named(..) value)."""
    if not json_object_prefix_ok(b):
        return False
    if choice == TOOL_NAMED:
        required = named
    elif choice == TOOL_REQUIRED:
        required = None
    else:
        return True
    r = json_name_so_far(b)
    if r[0] == "missing":
        return True
    if r[0] == "invalid":
        return False
    v = r[1]
    if r[0] == "partial":
        if required is not None:
            return required.startswith(v)
        return not names or any(nm.startswith(v) for nm in names)
    if required is not None:
        return v == required
    return not names or any(nm == v for nm in names)


def token_allowed(so_far: bytes, piece: bytes, c: dict) -> bool:
    """sample.rs:92-107. c: json_object (bool), tool_choice (TOOL_*), tool_name (bytes),
    tool_names (list of bytes), grammar (str or None)."""
    nxt = so_far + piece
    constrains = c.get("tool_choice", TOOL_NONE) in (TOOL_REQUIRED, TOOL_NAMED)
    if (c.get("json_object") or constrains) and not json_object_prefix_ok(nxt):
        return False
    if constrains and not tool_call_prefix_ok(nxt, c["tool_choice"], c.get("tool_name", b""),
                                              c.get("tool_names", [])):
        return False
    g = c.get("grammar")
    if g is not None:
        if parse_id_union(g) is not None:
            return True
        lit = parse_literal_root(g)
        if lit is not None:
            return lit.encode("utf-8").startswith(nxt)
    return True


def allow_mask(pieces, so_far: bytes, c: dict):
    """apply_constraint (sample.rs:63-90) as a list of allowed flags over the vocabulary
    (decode(i) = pieces[i]); the generated ids' pieces concatenate to so_far."""
    V = len(pieces)
    constrains = c.get("tool_choice", TOOL_NONE) in (TOOL_REQUIRED, TOOL_NAMED)
    g = c.get("grammar")
    if g is None and not c.get("json_object") and not constrains:
        return [True] * V
    if g is not None:
        u = parse_id_union(g)
        if u is not None:
            return [i in u for i in range(V)]
    return [token_allowed(so_far, pieces[i], c) for i in range(V)]


def pack_mask(flags):
    """Packed u32 words: bit id & 31 of word id >> 5."""
    import numpy as np

    V = len(flags)
    words = np.zeros((V + 31) // 32, np.uint32)
    for i, f in enumerate(flags):
        if f:
            words[i >> 5] |= np.uint32(1 << (i & 31))
    return words
