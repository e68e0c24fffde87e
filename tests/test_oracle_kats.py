"""Known-answer tests of the CPU oracle, restated from the reference's own unit tests.

Each test names the reference test it restates (crates/bfi-runtime/src/sample.rs:466-689,
engine/spec.rs:193-256, engine/decode_tests.rs:125-169). Inputs and expected outputs are
the reference's; `sample()` draws with u = Rng(seed).f32() exactly as sample.rs:307 does.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def S(logits, prev, seed=0, mask=None, **params):
    return O.sample_seeded(np.array(logits, np.float32), np.array(prev, np.uint32), params, seed, mask)


# ---- sample.rs:466-689 ------------------------------------------------------------------


def test_greedy_argmax():  # sample.rs:467
    assert S([1.0, 0.0, 0.5], [], temperature=0.0) == 0
    assert S([0.1, 2.0, 1.5], [], temperature=0.0) == 1


def test_default_is_greedy():  # sample.rs:477
    d = O.DEFAULTS
    assert d["temperature"] == 0.0 and d["top_k"] == 0 and d["top_p"] == 1.0
    assert d["min_p"] == 0.0 and d["repeat_penalty"] == 1.0 and d["presence_penalty"] == 0.0
    assert S([1.0, 0.0, 0.5], []) == 0


def test_sample_params_carries_grammar():  # sample.rs:495 (the id union parses)
    m = O.parse_id_union("root ::= id(1)", 3)
    assert m is not None and m[0] == 0b010


def test_grammar_id_mask_rejects_forbidden_token():  # sample.rs:506
    m = O.parse_id_union("root ::= id(1)", 3)
    assert S([9.0, 1.0, 8.0], [], temperature=0.0, mask=m) == 1


def _mask(allowed, V):
    m = np.zeros((V + 31) // 32, np.uint32)
    for i in allowed:
        m[i >> 5] |= np.uint32(1 << (i & 31))
    return m


def test_json_object_constraint_invoked_mask_half():  # sample.rs:517
    # decode(0) = "x" is not a JSON-object prefix, decode(1) = "{" is: the constraint
    # leaves only token 1, which is what the packed mask carries across the boundary.
    assert S([9.0, 1.0], [], temperature=0.0, mask=_mask([1], 2)) == 1


def test_required_tool_choice_forces_json_object_mask_half():  # sample.rs:531
    assert S([9.0, 1.0], [], temperature=0.0, mask=_mask([1], 2)) == 1


def test_named_tool_choice_rejects_other_name_mask_half():  # sample.rs:545
    assert S([9.0, 1.0], [], temperature=0.0, mask=_mask([1], 2)) == 1


def test_literal_grammar_stays_on_prefix_mask_half():  # sample.rs:563
    # so_far = "": "a" keeps the literal "ab" prefix, "z" and "b" do not
    assert S([1.0, 9.0, 2.0], [], temperature=0.0, mask=_mask([0], 3)) == 0
    # so_far = "a": only "b" continues it; history [0] carries no penalty by default
    assert S([1.0, 9.0, 2.0], [0], temperature=0.0, mask=_mask([2], 3)) == 2


def test_repeat_penalty_shifts_greedy():  # sample.rs:584
    assert S([1.2, 1.0], [0], temperature=0.0, repeat_penalty=1.5) == 1


def test_presence_penalty_subtracts():  # sample.rs:595
    assert S([1.0, 0.5], [0], temperature=0.0, presence_penalty=0.5) == 0


def test_temperature_scales_logits():  # sample.rs:608
    assert S([1.0, 100.0], [], temperature=10.0) <= 1
    assert S([1.0, 100.0], [], temperature=0.1) == 1


def test_top_k_filters():  # sample.rs:628
    assert S([10.0, 5.0, 2.0, 1.0], [], temperature=0.0, top_k=2) == 0


def test_top_k_with_temperature_never_picks_outside_k():  # sample.rs:641
    logits = [10.0, 9.0, 8.0, 7.0]
    for seed in range(32):
        assert S(logits, [], seed=seed, temperature=5.0, top_k=1) == 0
    for seed in range(32):
        assert S(logits, [], seed=seed, temperature=5.0, top_k=2) <= 1


def test_top_p_nucleus():  # sample.rs:667
    logits = [10.0, 5.0, 1.0, 0.1]
    assert S(logits, [], temperature=1.0, top_p=0.5) == 0
    assert S(logits, [], temperature=1.0, top_p=0.999) <= 3


# ---- engine/spec.rs:193-256 -------------------------------------------------------------


def test_draft_copies_what_followed_the_last_trigram():  # spec.rs:194
    ctx = [9, 1, 2, 3, 4, 5, 6, 7, 8, 1, 2, 3]
    assert O.draft(ctx, 4, 3, 2) == [4, 5, 6, 7]
    assert O.draft(ctx, 2, 3, 2) == [4, 5]
    assert O.draft(ctx, 0, 3, 2) == []


def test_draft_prefers_most_recent_match_and_falls_back_to_bigram():  # spec.rs:203
    ctx = [1, 2, 10, 11, 1, 2, 20, 21, 7, 1, 2]
    assert O.draft(ctx, 2, 3, 2) == [20, 21]
    assert O.draft([1, 2, 3, 4, 5], 4, 3, 2) == []
    assert O.draft([5, 6, 5, 6, 5, 6], 4, 3, 2) == [5, 6]


def test_greedy_judging_is_exact():  # spec.rs:214
    assert O.judge(("token", 7), 7, 0.99, 0.5) == ("accept", None)
    assert O.judge(("token", 7), 3, 0.0, 0.5) == ("reject", 7)


def test_sampled_judging_follows_target_probability():  # spec.rs:220
    t = ("weights", [(1, 0.75), (2, 0.25)])
    assert O.judge(t, 1, 0.5, 0.0) == ("accept", None)
    assert O.judge(t, 1, 0.9, 0.3) == ("reject", 2)
    assert O.judge(t, 9, 0.0, 0.0) == ("reject", 1)
    assert O.judge(("weights", [(4, 1.0)]), 4, 0.999999, 0.0) == ("accept", None)


def test_speculative_acceptance_preserves_distribution():  # spec.rs:233
    t = ("weights", [(0, 0.5), (1, 0.3), (2, 0.2)])
    state = 12345
    counts = [0, 0, 0]
    n = 60000
    for _ in range(n):
        u, state = O.rng_f32(state)
        u2, state = O.rng_f32(state)
        v = O.judge(t, 1, u, u2)
        counts[1 if v[0] == "accept" else v[1]] += 1
    for i, want in enumerate([0.5, 0.3, 0.2]):
        assert abs(counts[i] / n - want) < 0.015


# ---- Rng / slot_rng golden vectors ------------------------------------------------------


def test_rng_golden_vectors():
    g = json.load(open(os.path.join(GOLDEN, "rng_vectors.json")))
    for e in g["rng"]:
        state = int(e["seed"], 16)
        for word, u in zip(e["words"], e["u"]):
            s1 = state
            w, state = O.rng_next(state)
            assert w == int(word, 16)
            uu, _ = O.rng_f32(s1)
            assert np.float32(uu) == np.float32(u)
    for e in g["slot_rng"]:
        s = O.slot_rng_seed(int(e["seed"], 16), e["prompt_len"])
        assert s == int(e["state"], 16)
        for u in e["u"]:
            uu, s = O.rng_f32(s)
            assert np.float32(uu) == np.float32(u)


def test_rng_zero_u_seeds():
    # Rng(seed).f32() is exactly 0.0 for small seeds: sample() then returns the first
    # element of the scan order even if its weight is 0 (sample.rs:314-319).
    for seed in (1, 7, 42):
        assert O.rng_f32(seed)[0] == 0.0
    # u = 0 over index-order weights (no top-k/top-p): the first id, whatever its weight
    assert O.draw([5, 6, 7], [0.0, 0.5, 0.5], 0.0) == 5


# ---- decode_tests.rs: spec greedy == plain greedy on the toy model -----------------------


V_TOY = 6
CTX_TOY = 128


def _toy_rule(history):
    # decode_tests.rs:23-34 (KV toy: acc stays 0)
    n = len(history)
    last = history[-1] if history else 0
    cycle = [1, 2, 3, 4, 1, 1]
    nxt = (last + 2) % V_TOY if n % 5 == 0 else cycle[last]
    return nxt


def _toy_logits(history):
    v = np.zeros(V_TOY, np.float32)
    v[_toy_rule(history)] = 10.0
    return v


def _run_plain(prompt, params, max_tokens, seed=0):
    ids = list(prompt)
    u, _ = O.rng_f32(seed)
    out = []
    while len(out) < max_tokens:
        t = O.sample(_toy_logits(ids), ids, params, None, u)
        ids.append(t)
        out.append(t)
    return out


def _run_spec(prompt, params, max_tokens, k=4, seed=0):
    """take_token_spec (spec.rs:101-181) with the model replaced by the toy rule."""
    ids = list(prompt)
    prompt_len = len(prompt)
    u_sample, _ = O.rng_f32(seed)
    rng = O.slot_rng_seed(seed, prompt_len)
    pending = None
    stats = dict(passes=0, drafted=0, accepted=0)
    while len(ids) - prompt_len < max_tokens:
        t0 = pending if pending is not None else O.sample(_toy_logits(ids), ids, params, None, u_sample)
        pending = None
        ids.append(t0)
        if len(ids) - prompt_len >= max_tokens:
            break
        remaining = max_tokens - (len(ids) - prompt_len)
        room = CTX_TOY - len(ids)
        kk = min(k, remaining, room)
        drafted = O.draft(ids, kk, 3, 2)
        if not drafted:
            continue
        stats["passes"] += 1
        stats["drafted"] += len(drafted)
        rows = np.stack([_toy_logits(ids + drafted[:i]) for i in range(len(drafted) + 1)])
        u_pairs = []
        r = rng
        for _ in drafted:
            a, r = O.rng_f32(r)
            b, r = O.rng_f32(r)
            u_pairs += [a, b]
        acc, nxt = O.verify_seq(rows, params, ids, drafted, np.array(u_pairs, np.float32), u_sample)
        judged = min(acc + 1, len(drafted))
        for _ in range(2 * judged):
            _, rng = O.rng_f32(rng)
        accepted = 0
        for i in range(acc):
            ids.append(drafted[i])
            accepted += 1
            if len(ids) - prompt_len >= max_tokens:
                break
        stats["accepted"] += accepted
        if accepted == acc and acc < len(drafted):
            pending = nxt
    return ids[prompt_len:], stats


PROMPT = [1, 2, 3, 4, 1, 2, 3, 4, 1]


def test_spec_lookup_greedy_matches_plain_decode():  # decode_tests.rs:126
    params = dict(temperature=0.0)
    plain = _run_plain(PROMPT, params, 40)
    fast, st = _run_spec(PROMPT, params, 40)
    assert len(plain) == 40
    assert fast == plain
    assert st["passes"] > 0 and st["accepted"] > 0
    assert st["accepted"] < st["drafted"]
    assert st["passes"] < 40


def test_spec_lookup_respects_max_tokens():  # decode_tests.rs:151
    for mx in [1, 2, 3, 7]:
        out, _ = _run_spec(PROMPT, dict(temperature=0.0), mx, k=8)
        assert len(out) == mx


def test_spec_lookup_sampling_runs_to_length():  # decode_tests.rs:163
    out, _ = _run_spec(PROMPT, dict(temperature=0.8), 30, seed=7)
    assert len(out) == 30 and all(t < V_TOY for t in out)
