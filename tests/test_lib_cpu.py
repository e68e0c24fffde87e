"""CPU tests of the C-ABI library: it loads, exports every function include/bfi_sampler.h
and include/bfi_mask.h declare, its host-side helpers (Rng, slot_rng, draft, id-union parsing, spec replay) agree
with the oracle and the reference KATs, and argument errors come back as status codes.
No GPU work is launched here."""
import ctypes
import json
import os
import re

import numpy as np
import pytest

import bfi_smp
import oracle as O
import workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("bfi_sampler.h", "bfi_mask.h", "bfi_prefix.h")]
GOLDEN = os.path.join(ROOT, "tests", "golden")


def declared_functions():
    src = "".join(open(h).read() for h in HEADERS)
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(bfi_[a-z0-9_]+)\s*\(", src)))


def test_library_loads_and_exports_every_declared_symbol():
    L = bfi_smp.lib()
    names = declared_functions()
    assert len(names) >= 19
    for n in names:
        assert hasattr(L, n), n
    assert L.bfi_smp_abi_version() == 1


def test_rng_matches_golden_vectors():
    g = json.load(open(os.path.join(GOLDEN, "rng_vectors.json")))
    for e in g["rng"]:
        st = int(e["seed"], 16)
        for word, u in zip(e["words"], e["u"]):
            uu, _ = bfi_smp.rng_f32(st)
            w, st = bfi_smp.rng_next_u64(st)
            assert w == int(word, 16)
            assert np.float32(uu) == np.float32(u)
    for e in g["slot_rng"]:
        assert bfi_smp.slot_rng_seed(int(e["seed"], 16), e["prompt_len"]) == int(e["state"], 16)


def test_draft_matches_reference_kats_and_oracle():
    # spec.rs:194-211
    ctx = [9, 1, 2, 3, 4, 5, 6, 7, 8, 1, 2, 3]
    assert bfi_smp.draft(ctx, 4) == [4, 5, 6, 7]
    assert bfi_smp.draft(ctx, 2) == [4, 5]
    assert bfi_smp.draft(ctx, 0) == []
    assert bfi_smp.draft([1, 2, 10, 11, 1, 2, 20, 21, 7, 1, 2], 2) == [20, 21]
    assert bfi_smp.draft([1, 2, 3, 4, 5], 4) == []
    assert bfi_smp.draft([5, 6, 5, 6, 5, 6], 4) == [5, 6]
    rng = np.random.default_rng(5)
    for _ in range(300):
        c = rng.integers(0, 6, rng.integers(0, 40)).tolist()
        k = int(rng.integers(0, 6))
        nmax, nmin = int(rng.integers(1, 5)), int(rng.integers(0, 4))
        assert bfi_smp.draft(c, k, nmax, nmin) == O.draft(c, k, nmax, nmin)


# Rust's str::trim strips Unicode White_Space (sample.rs:231-235); code points a Rust
# program does not treat as whitespace (U+200B, U+180E, U+FEFF, the C0 separators U+001C..
# U+001F that Python's str.isspace accepts) must stay.
_WS_IN = ["\u00a0", "\u3000", "\u2028", "\u2029", "\u0085", "\u1680", "\u2000", "\u200a", "\u202f", "\u205f",
          "\x0b", "\x0c", "\t\u3000\n"]
_WS_OUT = ["\u200b", "\u180e", "\ufeff", "\x1c", "\x1f", "\u2060"]


def _id_union_cases():
    cases = ["root ::= id(1)", "  root ::=  id( 3 ) | id(+7)|id(0)  ", "root ::= id(1) | foo", 'root ::= "ab"',
             "root::=id(5)", "root ::= ", "root ::= id(4294967295)", "root ::= id(4294967296)", "rootx ::= id(1)",
             "root ::= id(70) | id(2)"]
    for w in _WS_IN + _WS_OUT:
        cases += [f"root ::= id(7){w}", f"{w}root ::= id(7)", f"root{w}::={w}id(7){w}|{w}id(9)",
                  f"root ::= id({w}12{w})", f"{w}{w}root ::= id(3) |id(4){w}{w}"]
    return cases


def test_parse_id_union_unicode_trim_matches_the_python_restatement():
    """bfi_parse_id_union and the C oracle against constraint.parse_id_union, whose trim is
    an independent statement of Rust's White_Space set."""
    import constraint as K
    for g in _id_union_cases():
        want = K.parse_id_union(g)
        a = bfi_smp.parse_id_union(g, 64)
        b = O.parse_id_union(g, 64)
        for got, who in ((a, "library"), (b, "oracle")):
            assert (got is None) == (want is None), (who, repr(g))
            if want is not None:
                ids = {i for i in range(64) if (int(got[i >> 5]) >> (i & 31)) & 1}
                assert ids == {i for i in want if i < 64}, (who, repr(g))
    # the whitespace set decides: these are id unions only with Rust's trim
    assert K.parse_id_union("root ::= id(7)\u3000") == {7}
    assert K.parse_id_union("root ::= id(7)\u200b") is None


def test_parse_id_union_matches_oracle():
    for g in _id_union_cases():
        a = bfi_smp.parse_id_union(g, 64)
        b = O.parse_id_union(g, 64)
        assert (a is None) == (b is None), repr(g)
        if a is not None:
            assert np.array_equal(a, b), repr(g)


def _py_replay(drafted, acc, nxt, eos, generated, max_tokens, rng_state, stops=None):
    """spec.rs:137-179 with push_token's rules (engine/mod.rs:451-462), restated for the
    comparison: two draws per judged draft; Reject -> correction; Eos -> done, not appended;
    Stopped (the draft completes a tool call) -> appended, counted, done; Continue ->
    appended, counted, then the budget."""
    pushed, accepted, done, correction = [], 0, False, None
    st = rng_state
    for i, d in enumerate(drafted):
        _, st = O.rng_f32(st)
        _, st = O.rng_f32(st)
        if i >= acc:
            correction = nxt
            break
        if eos is not None and d == eos:
            done = True
            break
        pushed.append(d)
        if stops is not None and stops[i]:
            accepted += 1
            done = True
            break
        accepted += 1
        if generated + len(pushed) >= max_tokens:
            done = True
            break
    return dict(pushed=pushed, accepted=accepted, done=done, pending=None if done else correction, rng_state=st)


def test_spec_replay_matches_stop_rules():
    rng = np.random.default_rng(11)
    for _ in range(600):
        n = int(rng.integers(0, 6))
        drafted = rng.integers(0, 5, n).tolist()
        acc = int(rng.integers(0, n + 1))
        nxt = int(rng.integers(0, 5))
        eos = None if rng.random() < 0.5 else int(rng.integers(0, 5))
        gen = int(rng.integers(1, 8))
        mx = gen + int(rng.integers(0, 6))
        st = int(rng.integers(0, 2**63))
        stops = None if rng.random() < 0.4 else (rng.random(n) < 0.3).tolist()
        got = bfi_smp.spec_replay(drafted, acc, nxt, eos, gen, mx, st, stops)
        want = _py_replay(drafted, acc, nxt, eos, gen, mx, st, stops)
        assert got == want


def test_spec_replay_tool_stop_ends_the_slot():
    """Pushed::Stopped (spec.rs:150-153): the draft that closes a tool call is appended and
    counted, the slot is done, later accepted drafts are dropped and no correction is
    pending; an EOS draft is never a stop (push_token checks EOS first)."""
    st = 12345
    r = bfi_smp.spec_replay([5, 6, 7, 8], 4, 9, None, 1, 100, st, [0, 1, 0, 0])
    assert r["pushed"] == [5, 6] and r["accepted"] == 2 and r["done"] and r["pending"] is None
    # every draft judged up to the stop draws twice: two judged drafts
    s2 = st
    for _ in range(4):
        _, s2 = O.rng_f32(s2)
    assert r["rng_state"] == s2
    # rejected before the stop: the correction stands
    r = bfi_smp.spec_replay([5, 6, 7], 1, 9, None, 1, 100, st, [0, 1, 0])
    assert r["pushed"] == [5] and not r["done"] and r["pending"] == 9
    # EOS wins over the stop flag
    r = bfi_smp.spec_replay([5, 3], 2, 9, 3, 1, 100, st, [0, 1])
    assert r["pushed"] == [5] and r["accepted"] == 1 and r["done"]
    # without the flags the old rules hold
    r = bfi_smp.spec_replay([5, 6, 7, 8], 4, 9, None, 1, 100, st)
    assert r["pushed"] == [5, 6, 7, 8] and not r["done"] and r["pending"] is None


def test_create_without_device_reports_error():
    # this container has no GPU: the C ABI must return a status, not crash
    try:
        import torch

        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except Exception:
        pass
    L = bfi_smp.lib()
    ctx = ctypes.c_void_p()
    rc = L.bfi_smp_create(0, ctypes.byref(ctx))
    assert rc != 0
    assert len(L.bfi_smp_last_error(None)) > 0
    # NULL context is rejected with a message
    rc = L.bfi_smp_sample_rows(None, None, 0, 1, 1, 1, None, None, None, None, 0, None, None, None)
    assert rc == 1 and b"ctx" in L.bfi_smp_last_error(None)


def test_workloads_are_deterministic_and_shaped():
    a = workloads.config("C2", seed=3, scale_v=0.05)
    b = workloads.config("C2", seed=3, scale_v=0.05)
    assert np.array_equal(a["logits"], b["logits"]) and np.array_equal(a["hist"], b["hist"])
    assert a["logits"].shape == (64, a["V"]) and a["hist_off"][-1] == 64 * 512
    c = workloads.config("C3", seed=1, scale_v=0.05)
    allowed = [int(np.unpackbits(c["mask"][r].view(np.uint8)).sum()) for r in range(c["B"])]
    assert allowed[0] == 1 and allowed[7] == 1 and min(allowed) >= 1
    d = workloads.config("C5", seed=1, scale_v=0.01)
    assert d["logits"].dtype == np.uint16 and d["B"] == 256


def test_c2_algorithmic_bytes_match_the_derivation():
    cfg = workloads.config("C2")
    B, V = 64, 151936
    # logits + 512-id histories + offsets + 32-byte params + u + token
    want = B * V * 4 + B * 512 * 4 + (B + 1) * 8 + B * 32 + B * 4 + B * 4
    assert workloads.algorithmic_bytes(cfg) == want


def test_mask_entry_points_reject_bad_arguments_without_a_device():
    """include/bfi_mask.h: argument errors come back as status codes (no GPU work)."""
    L = bfi_smp.lib()
    assert L.bfi_mask_error(None) == b"null context"
    assert L.bfi_mask_set_vocab(None, None, None, 0) == 1  # BFI_SMP_EINVAL
    c = bfi_smp.Constraint()
    assert L.bfi_mask_build(None, None, 0, ctypes.byref(c), None, None, None) == 1
    h = ctypes.c_void_p()
    rc = L.bfi_mask_create(-1, ctypes.byref(h))
    assert rc != 0 and not h.value
    L.bfi_mask_destroy(None)
