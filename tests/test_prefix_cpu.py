"""CPU tests of the prefix cache (include/bfi_prefix.h) in host-memory mode: the reference's own
unit tests (crates/bfi-runtime/src/engine/prefix.rs:392-498) restated as known answers and run
against both the library and the oracle restatement (oracle/prefix.py), then the library
against the oracle on random operation sequences (lookups, restores, inserts, evictions)."""
import numpy as np
import pytest

import bfi_smp
import prefix as OP


def kv_state(n):
    """prefix.rs:365-376: a KV-only state of n tokens, 1 layer, 2 floats a row, capacity 512."""
    data = np.zeros((512, 1, 2), np.float32)
    data.reshape(-1)[: n * 2] = np.arange(1, n * 2 + 1, dtype=np.float32)
    return n, [data, data.copy()], [None]


def recurrent_state(n):
    """prefix.rs:378-382."""
    n, kv, _ = kv_state(n)
    return n, kv, [np.full((1, 2, 2), 0.5, np.float32)]


LOGITS = np.array([0.1, 0.2], np.float32)  # prefix.rs:384-386


def seq(n, salt):  # prefix.rs:388-390
    return [i * 7 + salt for i in range(n)]


class Lib:
    """The library's cache with the oracle's calling convention."""

    def __init__(self, budget):
        self.c = bfi_smp.PrefixCache(budget, -1)

    def insert(self, tokens, state, logits=LOGITS):
        n, kv, rec = state
        self.c.insert(tokens, n, kv, rec, logits)

    def lookup(self, ids):
        return self.c.lookup(ids)

    def restore(self, hit, like):
        n, kv, rec = like
        kv = [np.full_like(t, -1.0) for t in kv]
        rec = [None if r is None else np.zeros_like(r) for r in rec]
        lg = np.zeros(2, np.float32)
        r = self.c.restore(hit, kv, rec, lg)
        if r is None:
            return None
        n, lr = r
        return n, kv, rec, (lg if lr else None)

    def __len__(self):
        return len(self.c)

    def used_bytes(self):
        return self.c.used_bytes()


class Orc:
    def __init__(self, budget):
        self.c = OP.PrefixCache(budget)

    def insert(self, tokens, state, logits=LOGITS):
        n, kv, rec = state
        self.c.insert(tokens, n, kv, rec, logits)

    def lookup(self, ids):
        return self.c.lookup(ids)

    def restore(self, hit, like):
        return self.c.restore(hit)

    def __len__(self):
        return len(self.c)

    def used_bytes(self):
        return self.c.used


BOTH = [Lib, Orc]


@pytest.mark.parametrize("impl", BOTH)
def test_exact_hit_restores_logits_and_compact_rows(impl):  # prefix.rs:393-409
    c = impl(1 << 20)
    ids = seq(5, 0)
    c.insert(ids, kv_state(5))
    hit = c.lookup(ids)
    assert hit[1:] == (5, 5)
    n, kv, rec, lg = c.restore(hit, kv_state(5))
    assert n == 5
    assert lg.tolist() == LOGITS.tolist()
    k = kv[0].reshape(-1)
    assert k.size == 1024  # restored at full capacity
    assert k[:10].tolist() == list(range(1, 11))
    assert (k[10:] == 0).all()
    assert c.used_bytes() < 200  # only the used rows are held


@pytest.mark.parametrize("impl", BOTH)
def test_longest_match_rewinds_inside_a_generated_entry(impl):  # prefix.rs:411-435
    c = impl(1 << 20)
    cached = seq(150, 0)
    c.insert(cached, kv_state(150))
    prompt = cached[:130] + [9999, 9998]
    hit = c.lookup(prompt)
    assert hit[1:] == (130, 130)
    n, kv, rec, lg = c.restore(hit, kv_state(150))
    assert n == 130 and lg is None  # logits are only known at the entry's end
    hit = c.lookup(cached[:100])
    assert hit[1:] == (100, 99)  # leave one token to forward for logits
    assert c.lookup([4242, 4243]) is None


@pytest.mark.parametrize("impl", BOTH)
def test_recurrent_entries_only_resume_at_their_end(impl):  # prefix.rs:437-454
    c = impl(1 << 20)
    cached = seq(80, 1)
    c.insert(cached, recurrent_state(80))
    assert c.lookup(cached[:70] + [1_000_000]) is None
    hit = c.lookup(cached + [5, 6])
    assert hit[1:] == (80, 80)
    n, kv, rec, lg = c.restore(hit, recurrent_state(80))
    assert rec[0] is not None and (rec[0] == 0.5).all()
    assert lg is not None


@pytest.mark.parametrize("impl", BOTH)
def test_evicts_least_recently_used_by_bytes(impl):  # prefix.rs:456-477
    c = impl(200)  # each 4-token entry: 16 B tokens + 8 B logits + 2 x 32 B rows = 88 B
    a, b, d = seq(4, 100), seq(4, 200), seq(4, 300)
    c.insert(a, kv_state(4))
    c.insert(b, kv_state(4))
    assert len(c) == 2
    c.restore(c.lookup(a), kv_state(4))  # touch a: b is now the least recently used
    c.insert(d, kv_state(4))
    assert len(c) == 2 and c.used_bytes() <= 200
    assert c.lookup(a) is not None
    assert c.lookup(b) is None
    assert c.lookup(d) is not None
    c.insert(seq(100, 7), kv_state(100))  # larger than the whole budget: not cached
    assert len(c) == 2


@pytest.mark.parametrize("impl", BOTH)
def test_extending_entry_supersedes_its_prefix(impl):  # prefix.rs:479-491
    c = impl(1 << 20)
    prompt = seq(10, 3)
    c.insert(prompt, kv_state(10))
    done = prompt + [1, 2, 3]
    c.insert(done, kv_state(13))
    assert len(c) == 1
    assert c.lookup(prompt)[1:] == (10, 9)


def test_forwarded_counter():  # prefix.rs:493-498
    c = bfi_smp.PrefixCache(1 << 30, -1)
    c.note_forward(3)
    c.note_forward(1)
    assert c.forwarded() == 4


def test_bytes_count_kept_rows_whole_tensors_and_recurrent_state():
    c = bfi_smp.PrefixCache(1 << 20, -1)
    k = np.ones((64, 8), np.float32)          # 32 B rows, 10 kept
    w = np.ones(100, np.uint8)                # a whole tensor (quantized storage)
    r = np.ones((3, 4), np.float32)           # recurrent, 48 B
    c.insert(list(range(10)), 10, [k, w], [r, None], np.ones(5, np.float32), whole=(1,))
    assert c.used_bytes() == 10 * 4 + 5 * 4 + 10 * 32 + 100 + 48
    # the state must cover exactly the tokens (prefix.rs:234): nothing cached otherwise
    c.insert(list(range(11)), 10, [k, w], [r, None], np.ones(5, np.float32), whole=(1,))
    assert len(c) == 1


def test_restore_rejects_a_layout_that_differs_from_the_entry():
    c = bfi_smp.PrefixCache(1 << 20, -1)
    n, kv, rec = kv_state(5)
    c.insert(seq(5, 0), n, kv, rec, LOGITS)
    hit = c.lookup(seq(5, 0))
    with pytest.raises(bfi_smp.SamplerError):
        c.restore(hit, [np.zeros((512, 1, 2), np.float32)], rec, np.zeros(2, np.float32))  # one K/V tensor short
    with pytest.raises(bfi_smp.SamplerError):
        c.restore(hit, [np.zeros((4, 1, 2), np.float32)] * 2, rec, np.zeros(2, np.float32))  # capacity below 5 rows
    with pytest.raises(bfi_smp.SamplerError):
        c.restore(hit, kv, rec, np.zeros(3, np.float32))  # logits of another size


def test_random_operation_sequences_match_the_oracle():
    """Random prompts over a small alphabet with shared prefixes across BLOCK boundaries, KV
    and recurrent states, lookups, restores and inserts under a tight byte budget: the same
    hits, the same restored contents, the same entry count and bytes after every step."""
    rng = np.random.default_rng(7)
    for trial in range(12):
        budget = int(rng.integers(2_000, 40_000))
        lib, orc = Lib(budget), Orc(budget)
        roots = [rng.integers(0, 4, int(rng.integers(1, 200))).tolist() for _ in range(4)]
        for step in range(120):
            root = roots[int(rng.integers(0, len(roots)))]
            cut = int(rng.integers(0, len(root) + 1))
            ids = root[:cut] + rng.integers(0, 4, int(rng.integers(0, 80))).tolist()
            op = rng.random()
            if op < 0.45:
                h1, h2 = lib.lookup(ids), orc.lookup(ids)
                assert (h1 is None) == (h2 is None), (trial, step, ids)
                if h1 is None:
                    continue
                assert h1[1:] == h2[1:], (trial, step)
                # the caller's tensors have the layout of the entry's kind
                like = kv_state(1) if orc.c.entries[h2[0]].rewindable else recurrent_state(1)
                got, want = lib.restore(h1, like), orc.restore(h2, like)
                assert (got is None) == (want is None)
                if want is None:
                    continue
                n_w, kv_w, rec_w, lg_w = want
                n_g, kv_g, rec_g, lg_g = got
                assert n_g == n_w
                for x, y in zip(kv_g, kv_w):
                    assert np.array_equal(x, y)
                assert (lg_g is None) == (lg_w is None)
                for x, y in zip(rec_g, rec_w):
                    assert (x is None) == (y is None) and (x is None or np.array_equal(x, y))
            elif ids:
                state = kv_state(min(len(ids), 512)) if rng.random() < 0.75 else recurrent_state(min(len(ids), 512))
                toks = ids[:state[0]]
                lib.insert(toks, state)
                orc.insert(toks, state)
            assert len(lib) == len(orc), (trial, step)
            assert lib.used_bytes() == orc.used_bytes(), (trial, step)
