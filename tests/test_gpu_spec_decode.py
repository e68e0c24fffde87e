"""Speculative decoding end to end on the GPU: engine/decode_tests.rs:125-169 restated over
the reference's toy model (decode_tests.rs:14-88), with every sampling decision made by the
HIP library through the C ABI: plain decode picks with bfi_smp_sample_host (sample.rs:304),
speculative decode drafts with bfi_draft (spec.rs:46-68), judges every draft of a step in
one bfi_smp_verify call over the forward_each rows (spec.rs:137-162) and replays the stop
rules with bfi_spec_replay (spec.rs:140-179). The engine loop around them (prefill, step,
take_token, take_token_spec with its state rollback, finish) is the reference's
(engine/mod.rs:349-430, spec.rs:101-181), restated here as test code."""
import numpy as np
import pytest

import bfi_smp

pytestmark = pytest.mark.gpu

V = 6
CTX = 128
PROMPT = [1, 2, 3, 4, 1, 2, 3, 4, 1]


def rule(history, acc):
    """decode_tests.rs:23-34: a 1->2->3->4->1 cycle broken every 5th position (and, for the
    recurrent toy, by the running sum)."""
    n = len(history)
    last = history[-1] if history else 0
    cycle = [1, 2, 3, 4, 1, 1]
    nxt = (last + 2) % V if n % 5 == 0 else cycle[last]
    if int(acc) % 7 == 3:
        nxt = (nxt + 1) % V
    return nxt


class Toy:
    """decode_tests.rs:36-88: the next token is a function of the whole history the state
    holds (KV rows, rewound by n), plus a running sum for the recurrent toy."""

    def __init__(self, recurrent):
        self.recurrent = recurrent

    def new_state(self):
        return dict(k=[0.0] * CTX, n=0, r=[0.0] if self.recurrent else None)

    def forward(self, tokens, state):
        assert state["n"] + len(tokens) <= CTX, "toy KV overflow"
        acc = 0.0
        for t in tokens:
            state["k"][state["n"]] = float(t)
            state["n"] += 1
            if self.recurrent:
                state["r"][0] = np.float32(state["r"][0] + np.float32(t))
                acc = state["r"][0]
        history = [int(x) for x in state["k"][:state["n"]]]
        values = np.zeros(V, np.float32)
        values[rule(history, acc)] = 10.0
        return values

    def forward_each(self, tokens, state):
        # rows[i] = logits after tokens[..=i] (arch.rs:40-60's default: one token at a time)
        return [self.forward([t], state) for t in tokens]


class Engine:
    def __init__(self, smp, recurrent, spec=None):
        self.smp, self.model, self.spec = smp, Toy(recurrent), spec
        self.stats = dict(verify_passes=0, drafted=0, accepted=0)

    # engine/mod.rs:349-400 (no prefix-cache hit: every test starts a fresh engine)
    def prefill_ids(self, ids, params):
        state = self.model.new_state()
        logits = self.model.forward(ids, state)
        mx = params["max_tokens"] if params["max_tokens"] else CTX - len(ids)
        return dict(all_ids=list(ids), prompt_len=len(ids), state=state, logits=logits, done=mx == 0,
                    max_tokens=mx, pending=None, rng=bfi_smp.slot_rng_seed(params.get("seed", 0), len(ids)))

    def budget_spent(self, slot):  # engine/mod.rs:425-430
        if len(slot["all_ids"]) - slot["prompt_len"] >= slot["max_tokens"]:
            slot["done"] = True
        return slot["done"]

    def pick(self, logits, slot, params):  # engine/mod.rs:445-447 on the GPU
        p = {k: params[k] for k in ("temperature",) if k in params}
        return self.smp.sample_seeded(logits, np.array(slot["all_ids"], np.uint32), p, params.get("seed", 0))

    def push_token(self, slot, tok):  # engine/mod.rs:451-462: no EOS, no tools in the toy
        slot["all_ids"].append(int(tok))
        return "continue"

    def take_token(self, slot, params):  # engine/mod.rs:410-422
        if self.budget_spent(slot):
            return
        nxt = self.pick(slot["logits"], slot, params)
        if self.push_token(slot, nxt) != "continue":
            return
        slot["logits"] = self.model.forward([nxt], slot["state"])
        self.budget_spent(slot)

    def take_token_spec(self, slot, params):  # spec.rs:101-181
        import torch

        spec = self.spec
        if self.budget_spent(slot):
            return
        t0 = slot["pending"] if slot["pending"] is not None else self.pick(slot["logits"], slot, params)
        slot["pending"] = None
        if self.push_token(slot, t0) != "continue":
            return
        n0 = slot["state"]["n"]
        remaining = max(slot["max_tokens"] - (len(slot["all_ids"]) - slot["prompt_len"]), 0)
        room = max(CTX - (n0 + 1), 0)
        k = min(spec["draft_len"], remaining, room)
        drafted = bfi_smp.draft(slot["all_ids"], k, spec["ngram_max"], spec["ngram_min"])
        if not drafted:
            slot["logits"] = self.model.forward([t0], slot["state"])
            self.budget_spent(slot)
            return
        tokens = [t0] + list(drafted)
        snapshot = None if slot["state"]["r"] is None else list(slot["state"]["r"])
        rows = self.model.forward_each(tokens, slot["state"])
        self.stats["verify_passes"] += 1
        self.stats["drafted"] += len(drafted)
        # one verify call over the k + 1 rows: uniforms from a copy of the slot RNG, two per
        # judged draft (spec.rs:142); the bonus row's uniform is pick()'s Rng(seed).f32()
        R = len(tokens)
        st, up = slot["rng"], []
        for _ in range(2 * len(drafted)):
            u, st = bfi_smp.rng_f32(st)
            up.append(u)
        ub, _ = bfi_smp.rng_f32(params.get("seed", 0))
        dev = "cuda:0"
        d_logits = torch.from_numpy(np.stack(rows)).to(dev)
        d_params = torch.from_numpy(bfi_smp.params_array([{"temperature": params.get("temperature", 0.0)}])
                                    .view(np.uint8).copy()).to(dev)
        hist = np.array(slot["all_ids"], np.uint32)
        d_hist = torch.from_numpy(hist.view(np.int32).copy()).to(dev)
        d_off = torch.tensor([0, hist.size], dtype=torch.int64, device=dev)
        d_drafts = torch.tensor(np.array(drafted, np.uint32).view(np.int32), device=dev).reshape(1, R - 1)
        d_dlen = torch.tensor([len(drafted)], dtype=torch.int32, device=dev)
        d_up = torch.tensor(up, dtype=torch.float32, device=dev)
        d_ub = torch.tensor([ub], dtype=torch.float32, device=dev)
        acc = torch.zeros(1, dtype=torch.int32, device=dev)
        nxt = torch.zeros(1, dtype=torch.int32, device=dev)
        self.smp.verify(d_logits, R, d_params, d_drafts, d_dlen, d_up, d_ub, acc, nxt, d_hist, d_off)
        torch.cuda.synchronize()
        gen = len(slot["all_ids"]) - slot["prompt_len"]
        r = bfi_smp.spec_replay(drafted, int(acc.item()), int(nxt.item()) & 0xFFFFFFFF, None, gen,
                                slot["max_tokens"], slot["rng"])
        slot["rng"] = r["rng_state"]
        slot["all_ids"].extend(r["pushed"])
        if r["done"]:
            slot["done"] = True
        accepted = r["accepted"]
        self.stats["accepted"] += accepted
        keep = n0 + 1 + accepted
        if keep < slot["state"]["n"]:  # spec.rs:164-175: roll the rejected drafts back
            if snapshot is not None:
                slot["state"]["r"] = snapshot
                slot["state"]["n"] = n0
                self.model.forward(tokens[:1 + accepted], slot["state"])
            else:
                slot["state"]["n"] = keep
        slot["logits"] = rows[accepted]
        if not slot["done"]:
            slot["pending"] = r["pending"]

    def step(self, slot, params):
        if self.spec is not None:
            self.take_token_spec(slot, params)
        else:
            self.take_token(slot, params)

    def run(self, prompt, params):  # decode_tests.rs:105-111
        slot = self.prefill_ids(prompt, params)
        while not slot["done"]:
            self.step(slot, params)
        return slot["all_ids"][slot["prompt_len"]:]


SPEC = dict(draft_len=4, ngram_max=3, ngram_min=2)  # SpecLookup::default (spec.rs:10-22)


def greedy(max_tokens):
    return dict(max_tokens=max_tokens, temperature=0.0)


@pytest.fixture(scope="module")
def smp(gpu):
    s = bfi_smp.Sampler(0)
    yield s
    s.close()


def test_spec_lookup_greedy_matches_plain_decode_kv_state(smp):
    params = greedy(40)
    plain = Engine(smp, False).run(PROMPT, params)
    e = Engine(smp, False, SPEC)
    fast = e.run(PROMPT, params)
    assert len(plain) == 40
    assert fast == plain, "speculative greedy must be token-identical"
    st = e.stats
    assert st["verify_passes"] > 0 and st["accepted"] > 0, st
    assert st["accepted"] < st["drafted"], st  # the toy breaks the cycle: some drafts rejected
    assert st["verify_passes"] < 40


def test_spec_lookup_rolls_back_recurrent_state(smp):
    params = greedy(40)
    plain = Engine(smp, True).run(PROMPT, params)
    e = Engine(smp, True, SPEC)
    fast = e.run(PROMPT, params)
    assert fast == plain, "recurrent rollback must restore the snapshot exactly"
    assert e.stats["accepted"] > 0


def test_spec_lookup_respects_max_tokens_and_context(smp):
    for mx in (1, 2, 3, 7):
        e = Engine(smp, False, dict(SPEC, draft_len=8))
        assert len(e.run(PROMPT, greedy(mx))) == mx
    out = Engine(smp, False, SPEC).run(PROMPT, greedy(CTX - len(PROMPT) - 1))
    assert len(out) == CTX - len(PROMPT) - 1


def test_spec_lookup_sampling_runs_to_length(smp):
    params = dict(max_tokens=30, temperature=0.8, seed=7)
    out = Engine(smp, False, SPEC).run(PROMPT, params)
    assert len(out) == 30
    assert all(t < V for t in out)
