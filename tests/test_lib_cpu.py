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
HEADERS = [os.path.join(ROOT, "include", h) for h in ("bfi_sampler.h", "bfi_mask.h")]
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


def test_parse_id_union_matches_oracle():
    cases = ["root ::= id(1)", "  root ::=  id( 3 ) | id(+7)|id(0)  ", "root ::= id(1) | foo", 'root ::= "ab"',
             "root::=id(5)", "root ::= ", "root ::= id(4294967295)", "root ::= id(4294967296)", "rootx ::= id(1)",
             "root ::= id(70) | id(2)"]
    for g in cases:
        a = bfi_smp.parse_id_union(g, 64)
        b = O.parse_id_union(g, 64)
        assert (a is None) == (b is None), g
        if a is not None:
            assert np.array_equal(a, b), g


def _py_replay(drafted, acc, nxt, eos, generated, max_tokens, rng_state):
    """spec.rs:140-179 stop rules, restated for the comparison."""
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
        accepted += 1
        if generated + len(pushed) >= max_tokens:
            done = True
            break
    return dict(pushed=pushed, accepted=accepted, done=done, pending=None if done else correction, rng_state=st)


def test_spec_replay_matches_stop_rules():
    rng = np.random.default_rng(11)
    for _ in range(400):
        n = int(rng.integers(0, 6))
        drafted = rng.integers(0, 5, n).tolist()
        acc = int(rng.integers(0, n + 1))
        nxt = int(rng.integers(0, 5))
        eos = None if rng.random() < 0.5 else int(rng.integers(0, 5))
        gen = int(rng.integers(1, 8))
        mx = gen + int(rng.integers(0, 6))
        st = int(rng.integers(0, 2**63))
        got = bfi_smp.spec_replay(drafted, acc, nxt, eos, gen, mx, st)
        want = _py_replay(drafted, acc, nxt, eos, gen, mx, st)
        assert got == want


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
