"""Pins the constraint oracle (oracle/constraint.py) before it checks the GPU mask producer:
the reference's own constraint tests (sample.rs:505-581) as known answers, Python's json
module on complete objects and on all their prefixes, hand-derived cases of the `"name"` scan
(sample.rs:144-206), and the grammar parsers (sample.rs:208-234). No GPU."""
import json
import random

import constraint as K


def allowed(pieces, so_far, **c):
    return K.allow_mask(pieces, so_far, c)


# ---- sample.rs:505-581 -------------------------------------------------------------------


def test_reference_grammar_id_mask():
    # sample.rs:506-514: only id 1 survives "root ::= id(1)"
    assert allowed([b"a", b"b", b"c"], b"", grammar="root ::= id(1)") == [False, True, False]


def test_reference_json_object_constraint():
    # sample.rs:517-528: "x" is an illegal first char, "{" is allowed
    assert allowed([b"x", b"{"], b"", json_object=True) == [False, True]


def test_reference_required_tool_choice():
    # sample.rs:531-542
    assert allowed([b"x", b"{"], b"", tool_choice=K.TOOL_REQUIRED, tool_names=[b"lookup"]) == [False, True]


def test_reference_named_tool_choice():
    # sample.rs:545-559
    pieces = [b'{"name":"other"}', b'{"name":"lookup"}']
    got = allowed(pieces, b"", tool_choice=K.TOOL_NAMED, tool_name=b"lookup", tool_names=[b"lookup", b"other"])
    assert got == [False, True]


def test_reference_literal_grammar():
    # sample.rs:562-581
    g = 'root ::= "ab"'
    assert allowed([b"a", b"z", b"b"], b"", grammar=g) == [True, False, False]
    assert allowed([b"a", b"z", b"b"], b"a", grammar=g) == [False, False, True]


def test_unconstrained_and_other_grammars_allow_everything():
    assert allowed([b"x", b"{"], b"") == [True, True]
    assert allowed([b"x", b"{"], b"", grammar="root ::= foo") == [True, True]


# ---- json_object_prefix_ok against the json module ---------------------------------------


def _rand_value(rng, depth):
    r = rng.random()
    if depth > 3 or r < 0.3:
        return rng.choice([1, -2.5, True, None, "s", 'q"uo\\te', "é✓", "", "{[}]", "name"])
    if r < 0.65:
        return {rng.choice(["a", "name", "b c", '"k"', "{"]): _rand_value(rng, depth + 1) for _ in range(rng.randint(0, 3))}
    return [_rand_value(rng, depth + 1) for _ in range(rng.randint(0, 3))]


def test_json_object_prefix_ok_accepts_every_prefix_of_an_object():
    rng = random.Random(7)
    for _ in range(300):
        obj = {"k%d" % i: _rand_value(rng, 1) for i in range(rng.randint(0, 4))}
        text = json.dumps(obj, ensure_ascii=rng.random() < 0.5, indent=rng.choice([None, 1]))
        b = (" " * rng.randint(0, 2) + text).encode()
        json.loads(b)  # a valid object
        for i in range(len(b) + 1):
            assert K.json_object_prefix_ok(b[:i]), b[:i]
        assert K.json_object_prefix_ok(b + b" \n\t\r\x0c")
        assert not K.json_object_prefix_ok(b + b"x")
        assert not K.json_object_prefix_ok(b + b"\x0b")  # \v is not is_ascii_whitespace
        assert not K.json_object_prefix_ok(b + b"}")


def test_json_object_prefix_ok_rejects_non_objects():
    for v in ([1, 2], "s", 3, None, True):
        assert not K.json_object_prefix_ok(json.dumps(v).encode())
    assert K.json_object_prefix_ok(b"")
    assert K.json_object_prefix_ok(b" \t\n")
    assert not K.json_object_prefix_ok(b"\x0b{")
    assert not K.json_object_prefix_ok(b"{]]")  # depth below zero
    assert K.json_object_prefix_ok(b'{"a": "}')  # the brace is inside a string
    assert K.json_object_prefix_ok(b'{"a": "\\')  # open escape
    assert not K.json_object_prefix_ok(b"{]x")  # ']' closes like '}' (brace/string scan only)
    assert K.json_object_prefix_ok(b"{]  ")


# ---- json_name_so_far / tool_call_prefix_ok ----------------------------------------------


def test_name_scan_cases():
    f = K.json_name_so_far
    assert f(b"") == ("missing",)
    assert f(b'{"name"') == ("missing",)
    assert f(b'{"name"  ') == ("missing",)
    assert f(b'{"name":') == ("partial", b"")
    assert f(b'{"name": "lo') == ("partial", b"lo")
    assert f(b'{"name" :\t"lookup"}') == ("complete", b"lookup")
    assert f(b'{"name": 5') == ("invalid",)
    assert f(b'{"name"x, "name": "a') == ("partial", b"a")  # not a key: the scan resumes
    assert f(b'{"name""name": "b"}') == ("complete", b"b")  # the closing quote starts a key
    assert f(b'{"name" "name": "c"}') == ("complete", b"c")
    assert f(b'{"x": "\\"name\\": \\"q') == ("missing",)  # escaped quotes do not form the key
    assert f(b'{"name": "a\\"b"}') == ("complete", b'a\\"b')  # escapes kept in the value
    assert f(b'{"name": "a\\') == ("partial", b"a\\")


def test_tool_call_prefix_cases():
    ok = K.tool_call_prefix_ok
    names = [b"lookup", b"list"]
    assert ok(b'{"name": "l', K.TOOL_REQUIRED, b"", names)
    assert ok(b'{"name": "lis', K.TOOL_REQUIRED, b"", names)
    assert not ok(b'{"name": "lx', K.TOOL_REQUIRED, b"", names)
    assert ok(b'{"name": "list"', K.TOOL_REQUIRED, b"", names)
    assert not ok(b'{"name": "lis"', K.TOOL_REQUIRED, b"", names)
    assert ok(b'{"name": "anything"', K.TOOL_REQUIRED, b"", [])
    assert ok(b'{"name": "look', K.TOOL_NAMED, b"lookup", names)
    assert not ok(b'{"name": "list', K.TOOL_NAMED, b"lookup", names)
    assert ok(b'{"name": "lookup"}', K.TOOL_NAMED, b"lookup", names)
    assert not ok(b'{"name": "lookupx"', K.TOOL_NAMED, b"lookup", names)
    assert not ok(b'{"name": 1', K.TOOL_NAMED, b"lookup", names)
    assert not ok(b'x{"name": "lookup"', K.TOOL_NAMED, b"lookup", names)  # not a JSON object
    assert ok(b'{"name": "zzz"', K.TOOL_AUTO, b"", names)  # auto does not constrain


# ---- grammar parsers ---------------------------------------------------------------------


def test_grammar_parsers():
    assert K.parse_id_union("root ::= id(1) | id( 2 ) |id(+3)") == {1, 2, 3}
    assert K.parse_id_union("  root::=id(7)　") == {7}
    assert K.parse_id_union("root ::= id(1) | x") is None
    assert K.parse_id_union("root ::= id(-1)") is None
    assert K.parse_id_union("root ::= id(4294967296)") is None
    assert K.parse_id_union("root ::= id()") is None
    assert K.parse_id_union("rot ::= id(1)") is None
    assert K.parse_literal_root('root ::= "ab"') == "ab"
    assert K.parse_literal_root('root ::= "a"b"') == "a"
    assert K.parse_literal_root('root ::= ab') is None
    assert K.parse_literal_root('root ::= "ab') is None
    assert K.rust_trim("\x1c a \x1c") == "\x1c a \x1c"  # not White_Space in Rust (Python strips it)


# ---- brute force against an independent statement of the brace/string scan --------------


def _prefix_ok_independent(b: bytes) -> bool:
    """json_object_prefix_ok stated differently: strings (closed, or open at the end) collapse
    to one byte by a regular expression, then the running bracket depth over what is left
    must stay positive until it first returns to zero, after which only ASCII whitespace may
    follow."""
    import itertools
    import re

    s = b.lstrip(b" \t\n\x0c\r")
    if not s:
        return True
    if s[:1] != b"{":
        return False
    t = re.sub(rb'"(?:\\.|\\$|[^"\\])*(?:"|$)', b"S", s, flags=re.S)
    steps = [1 if c in b"{[" else -1 if c in b"}]" else 0 for c in t]
    depth = list(itertools.accumulate(steps))
    for i, d in enumerate(depth):
        if d <= 0:
            return all(c in b" \t\n\x0c\r" for c in t[i + 1:])
    return True


def test_json_object_prefix_ok_brute_force():
    import itertools

    alphabet = [b" ", b"{", b"}", b"[", b"]", b'"', b"\\", b"a", b"\x0b"]
    n = 0
    for length in range(0, 7):
        for combo in itertools.product(alphabet, repeat=length):
            b = b"".join(combo)
            assert K.json_object_prefix_ok(b) == _prefix_ok_independent(b), b
            n += 1
    assert n > 500000


# ---- json_name_so_far / tool_call_prefix_ok against an independent statement ------------
#
# sample.rs:144-206 as a search over regular expressions rather than a byte loop: every
# start of `"name"` (overlapping starts included: the closing quote may open the next key),
# in order; blanks are u8::is_ascii_whitespace (space, \t, \n, \x0c, \r).

import re

_BL = rb"[ \t\n\x0c\r]*"
_KEY = re.compile(rb'(?="name")')
_AFTER_KEY = re.compile(_BL + rb"(:?)")
_VALUE = re.compile(rb"((?:[^\"\\]|\\[\x00-\xff])*)(\\?)(\"?)", re.S)


def _name_so_far_independent(b: bytes):
    for m in _KEY.finditer(b):
        j = m.start() + 6
        a = _AFTER_KEY.match(b, j)
        if a.end() == len(b) and not a.group(1):
            return ("missing",)  # blanks run to the end: no colon yet
        if not a.group(1):
            continue  # not followed by a colon: not the key, keep looking
        k = re.compile(_BL).match(b, a.end()).end()
        if k == len(b):
            return ("partial", b"")
        if b[k:k + 1] != b'"':
            return ("invalid",)
        v = _VALUE.match(b, k + 1)
        body = v.group(1) + v.group(2)  # a trailing lone backslash stays in the value
        return ("complete", body) if v.group(3) else ("partial", body)
    return ("missing",)


def _tool_ok_independent(b: bytes, choice: int, named: bytes, names) -> bool:
    if not _prefix_ok_independent(b):
        return False
    if choice not in (K.TOOL_REQUIRED, K.TOOL_NAMED):
        return True
    kind, *val = _name_so_far_independent(b)
    allowed = [named] if choice == K.TOOL_NAMED else list(names)
    if kind == "missing":
        return True
    if kind == "invalid":
        return False
    v = val[0]
    if choice == K.TOOL_REQUIRED and not names:
        return True
    if kind == "partial":
        return any(n[:len(v)] == v for n in allowed)
    return v in allowed


def _name_strings():
    import itertools

    # everything up to 5 bytes over the key's and value's bytes, and every string of the form
    # <up to 2 bytes> "name" <up to 5 bytes> over the bytes that decide the scan
    full = [b'"', b"n", b"a", b":", b"\\", b" ", b"x"]
    for length in range(0, 6):
        for combo in itertools.product(full, repeat=length):
            yield b"".join(combo)
    pre = [b'"', b"x", b" "]
    post = [b'"', b":", b"\\", b" ", b"\t", b"l", b"x"]
    heads = [b""] + [b"".join(c) for k in (1, 2) for c in itertools.product(pre, repeat=k)]
    tails = [b"".join(c) for k in range(0, 6) for c in itertools.product(post, repeat=k)]
    for h in heads:
        for t in tails:
            yield h + b'"name"' + t
            yield b"{" + h + b'"name"' + t
    # a second key after the first (the scan resumes after a non-colon; the first key's
    # closing quote can open the second)
    short = [t for t in tails if len(t) <= 3]
    for h in heads[:4]:
        for mid in (b"", b" ", b"x", b":", b'"', b"name"):
            for t in short:
                yield b"{" + h + b'"name"' + mid + b'"name"' + t


def test_json_name_so_far_brute_force():
    n = 0
    for b in _name_strings():
        assert K.json_name_so_far(b) == _name_so_far_independent(b), b
        n += 1
    assert n > 100000


def test_tool_call_prefix_ok_brute_force():
    names = [b"l", b"lx", b'l"']
    n = 0
    for b in _name_strings():
        if not b.startswith(b"{"):
            b = b"{" + b
        for choice, named, nm in ((K.TOOL_REQUIRED, b"", names), (K.TOOL_REQUIRED, b"", []),
                                  (K.TOOL_NAMED, b"lx", names), (K.TOOL_AUTO, b"", names)):
            assert K.tool_call_prefix_ok(b, choice, named, nm) == _tool_ok_independent(b, choice, named, nm), (b, choice)
            n += 1
    assert n > 100000
