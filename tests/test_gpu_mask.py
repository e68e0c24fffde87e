"""GPU parity of the allow-mask producer (include/bfi_mask.h) against the constraint oracle
(oracle/constraint.py, a restatement of sample.rs:63-291): every mask word must be equal.
Cases: the reference's constraint tests (sample.rs:505-581), small vocabularies of
structural pieces under every prefix of tool-call texts for json_object / required / named
tool choices and literal grammars, tool-name tables (names that prefix each other, 64
names), id unions, a full 151,936-piece vocabulary, and pieces of thousands of bytes."""
import random

import numpy as np
import pytest

import bfi_smp
import constraint as K

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mp(gpu):
    m = bfi_smp.MaskProducer(0)
    yield m
    m.close()


def gpu_mask(mp, so_far, c):
    import torch

    nw = (mp.V + 31) // 32
    d = torch.full((max(nw, 1),), -1, dtype=torch.int32, device="cuda")  # poisoned
    flag = mp.build(so_far, d, **c)
    torch.cuda.synchronize()
    return d.cpu().numpy().view(np.uint32)[:nw], flag


def check(mp, pieces, so_far, name="", **c):
    if mp.V != len(pieces) or getattr(mp, "_pieces", None) is not pieces:
        mp.set_vocab(pieces)
        mp._pieces = pieces
    print(f"[mask] {name} V={len(pieces)} so_far={so_far[:40]!r} {c}", flush=True)
    got, flag = gpu_mask(mp, so_far, c)
    exp = K.pack_mask(K.allow_mask(pieces, so_far, c))
    if not np.array_equal(got, exp):
        w = int(np.argmax(got != exp))
        bad = [i for i in range(w * 32, min(w * 32 + 32, len(pieces))) if ((got[w] ^ exp[w]) >> (i & 31)) & 1]
        raise AssertionError(f"{name}: mask differs at ids {bad[:8]} pieces {[pieces[i] for i in bad[:4]]} "
                             f"so_far={so_far!r} c={c}")
    return flag


def test_reference_constraint_kats(mp):
    # sample.rs:505-581
    assert check(mp, [b"a", b"b", b"c"], b"", "id-union", grammar="root ::= id(1)") == 1
    check(mp, [b"x", b"{"], b"", "json", json_object=True)
    check(mp, [b"x", b"{"], b"", "required", tool_choice=K.TOOL_REQUIRED, tool_names=[b"lookup"])
    check(mp, [b'{"name":"other"}', b'{"name":"lookup"}'], b"", "named", tool_choice=K.TOOL_NAMED,
          tool_name=b"lookup", tool_names=[b"lookup", b"other"])
    for sf in (b"", b"a", b"ab", b"b"):
        check(mp, [b"a", b"z", b"b"], sf, "literal", grammar='root ::= "ab"')
    assert check(mp, [b"x", b"{"], b"", "unconstrained") == 0


FRAGS = [b"{", b"}", b"[", b"]", b'"', b"\\", b":", b" ", b"\t", b"\n", b"\x0b", b"\x0c", b",", b"name", b'"name"',
         b'"nam', b'e"', b"a", b"l", b"lookup", b"list", b"lis", b"x", b'"}', b'{"', b' "', "é".encode(), b'\\"',
         b"arguments", b"1", b"hel", b"lo", b" wor", b"ld", b"hello world"]


def rand_pieces(rng, V):
    out = []
    for _ in range(V):
        out.append(b"".join(rng.choice(FRAGS) for _ in range(rng.randint(1, 3))))
    out[0] = b""
    return out


TEXTS = [
    b'{"name": "lookup", "arguments": {"q": "a\\"b", "n": [1, {"x": "}"}]}}  ',
    b'  {"name" "name":"list"}',
    b'{"x": "\\"name\\": \\"z", "name"x, "name":\t"lis',
    b'{"name": 5}',
    b'[{"name": "lookup"}]',
]


def test_random_vocabularies_over_text_prefixes(mp):
    rng = random.Random(11)
    pieces = rand_pieces(rng, 700)
    names = [b"lookup", b"list", b"lis", b"listing", b"x"]
    variants = [
        dict(json_object=True),
        dict(tool_choice=K.TOOL_REQUIRED, tool_names=names),
        dict(tool_choice=K.TOOL_REQUIRED, tool_names=[]),
        dict(tool_choice=K.TOOL_NAMED, tool_name=b"lookup", tool_names=names),
        dict(tool_choice=K.TOOL_NAMED, tool_name=b"lis", tool_names=[]),
        dict(tool_choice=K.TOOL_AUTO, tool_names=names, json_object=True),
    ]
    for t, text in enumerate(TEXTS):
        for cut in range(0, len(text) + 1, 3):
            for v, c in enumerate(variants):
                check(mp, pieces, text[:cut], f"text{t}-cut{cut}-v{v}", **c)


def test_literal_grammars_and_id_unions(mp):
    rng = random.Random(12)
    pieces = rand_pieces(rng, 500)
    lit = "hello world"
    for cut in range(len(lit) + 2):
        so_far = (lit + "!").encode()[:cut]
        check(mp, pieces, so_far, f"literal-{cut}", grammar=f'root ::= "{lit}"')
        check(mp, pieces, so_far, f"literal-json-{cut}", grammar=f'root ::= "{lit}"', json_object=True)
    check(mp, pieces, b"", "literal-empty", grammar='root ::= ""')
    check(mp, pieces, b"", "id-union", grammar="root ::= id(0) | id(+31) | id(32) | id(499) | id(9999)")
    check(mp, pieces, b"{", "id-union-wins-over-json", grammar="root ::= id(3)", json_object=True)
    check(mp, pieces, b"{", "other-grammar", grammar="root ::= thing", json_object=True)


def test_tool_name_tables(mp):
    rng = random.Random(13)
    names = [("t%02d" % i).encode() for i in range(63)] + [b"lookup"]
    pieces = rand_pieces(rng, 300) + [b"t0", b"t01", b"t01\"", b"t63", b'lookup"', b"lookupx", b'"t', b'"l']
    for so_far in (b'{"name": "', b'{"name": "t', b'{"name": "t0', b'{"name":"lookup'):
        check(mp, pieces, so_far, "64-names", tool_choice=K.TOOL_REQUIRED, tool_names=names)
        check(mp, pieces, so_far, "named-t01", tool_choice=K.TOOL_NAMED, tool_name=b"t01", tool_names=names)
    with pytest.raises(bfi_smp.SamplerError):
        check(mp, pieces, b"", "65-names", tool_choice=K.TOOL_REQUIRED, tool_names=names + [b"one-more"])


def test_full_vocabulary(mp):
    rng = random.Random(14)
    pieces = rand_pieces(rng, 151936)
    check(mp, pieces, b'{"name": "lo', "full-named", tool_choice=K.TOOL_NAMED, tool_name=b"lookup",
          tool_names=[b"lookup", b"list"])
    check(mp, pieces, b'{"name": "lookup", "arguments": {"q": "', "full-json", json_object=True)


def test_long_pieces(mp):
    """Pieces of thousands of bytes (read from the text, not the 16-byte rows), an empty
    vocabulary slot, and a 3000-byte literal (its tail, cut to the longest piece, travels in
    the kernel arguments)."""
    rng = random.Random(15)
    pieces = rand_pieces(rng, 600)
    for i in range(0, 600, 37):
        body = b"".join(rng.choice([b" ", b"{", b"}", b'"', b"\\", b"name", b'"name": "l', b"x"]) for _ in range(900))
        pieces[i] = body
    pieces[5] = b""
    for so_far in (b"", b"{", b'{"name": "l', b'{"a": "'):
        check(mp, pieces, so_far, "long-json", json_object=True)
        check(mp, pieces, so_far, "long-named", tool_choice=K.TOOL_NAMED, tool_name=b"lookup", tool_names=[b"lookup"])
    lit = "{" * 3000
    check(mp, pieces, b"{{", "long-literal", grammar=f'root ::= "{lit}"')
