"""GPU tests of the prefix cache with its entries in device memory (include/bfi_prefix.h): the
reference's own unit tests (crates/bfi-runtime/src/engine/prefix.rs:392-498) on device
tensors, a larger K/V state whose rows must come back byte for byte with the tail zeroed, and
the oracle restatement (oracle/prefix.py) compared with the device cache on random operation
sequences."""
import numpy as np
import pytest

import bfi_smp
import prefix as OP

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def kv_state(n, cap=512):
    data = np.zeros((cap, 1, 2), np.float32)
    data.reshape(-1)[: n * 2] = np.arange(1, n * 2 + 1, dtype=np.float32)
    return n, [data, data.copy()], [None]


def recurrent_state(n):
    n, kv, _ = kv_state(n)
    return n, kv, [np.full((1, 2, 2), 0.5, np.float32)]


LOGITS = np.array([0.1, 0.2], np.float32)


def seq(n, salt):
    return [i * 7 + salt for i in range(n)]


class DevCache:
    """The device cache with host arrays in and out (copied to and from the GPU around it)."""

    def __init__(self, budget):
        self.c = bfi_smp.PrefixCache(budget, 0)

    def insert(self, tokens, state, logits=LOGITS):
        import torch

        n, kv, rec = state
        s = torch.cuda.current_stream()
        self.c.insert(tokens, n, [_dev(t) for t in kv], [None if r is None else _dev(r) for r in rec], _dev(logits),
                      stream=s.cuda_stream)
        s.synchronize()

    def lookup(self, ids):
        return self.c.lookup(ids)

    def restore(self, hit, like):
        import torch

        n, kv, rec = like
        kv_d = [_dev(np.full_like(t, -1.0)) for t in kv]
        rec_d = [None if r is None else _dev(np.zeros_like(r)) for r in rec]
        lg = _dev(np.zeros(2, np.float32))
        s = torch.cuda.current_stream()
        r = self.c.restore(hit, kv_d, rec_d, lg, stream=s.cuda_stream)
        s.synchronize()
        if r is None:
            return None
        n, lr = r
        return (n, [t.cpu().numpy() for t in kv_d], [None if t is None else t.cpu().numpy() for t in rec_d],
                lg.cpu().numpy() if lr else None)

    def __len__(self):
        return len(self.c)

    def used_bytes(self):
        return self.c.used_bytes()


def test_reference_kats_on_device(gpu):
    # prefix.rs:393-409
    c = DevCache(1 << 20)
    ids = seq(5, 0)
    c.insert(ids, kv_state(5))
    hit = c.lookup(ids)
    assert hit[1:] == (5, 5)
    n, kv, rec, lg = c.restore(hit, kv_state(5))
    k = kv[0].reshape(-1)
    assert n == 5 and lg.tolist() == LOGITS.tolist()
    assert k[:10].tolist() == list(range(1, 11)) and (k[10:] == 0).all()
    assert c.used_bytes() < 200
    # prefix.rs:411-435
    c = DevCache(1 << 20)
    cached = seq(150, 0)
    c.insert(cached, kv_state(150))
    hit = c.lookup(cached[:130] + [9999, 9998])
    assert hit[1:] == (130, 130)
    n, kv, rec, lg = c.restore(hit, kv_state(150))
    assert n == 130 and lg is None
    assert c.lookup(cached[:100])[1:] == (100, 99)
    assert c.lookup([4242, 4243]) is None
    # prefix.rs:437-454
    c = DevCache(1 << 20)
    cached = seq(80, 1)
    c.insert(cached, recurrent_state(80))
    assert c.lookup(cached[:70] + [1_000_000]) is None
    hit = c.lookup(cached + [5, 6])
    assert hit[1:] == (80, 80)
    n, kv, rec, lg = c.restore(hit, recurrent_state(80))
    assert (rec[0] == 0.5).all() and lg is not None
    # prefix.rs:456-477
    c = DevCache(200)
    a, b, d = seq(4, 100), seq(4, 200), seq(4, 300)
    c.insert(a, kv_state(4))
    c.insert(b, kv_state(4))
    c.restore(c.lookup(a), kv_state(4))
    c.insert(d, kv_state(4))
    assert len(c) == 2 and c.used_bytes() <= 200
    assert c.lookup(a) is not None and c.lookup(b) is None and c.lookup(d) is not None
    c.insert(seq(100, 7), kv_state(100))
    assert len(c) == 2
    # prefix.rs:479-491
    c = DevCache(1 << 20)
    prompt = seq(10, 3)
    c.insert(prompt, kv_state(10))
    c.insert(prompt + [1, 2, 3], kv_state(13))
    assert len(c) == 1 and c.lookup(prompt)[1:] == (10, 9)


def test_large_state_rows_come_back_exactly(gpu):
    """Four K/V layers of [2048 positions, 8 heads, 128] bf16-sized rows (as int16 bit patterns)
    and a 1 MiB recurrent tensor: the kept rows equal the inserted ones, the rest is zero."""
    import torch

    rng = np.random.default_rng(3)
    n = 1500
    kv = [rng.integers(-32768, 32767, (2048, 8, 128), dtype=np.int16) for _ in range(4)]
    rec = [None, rng.integers(0, 255, 1 << 20, dtype=np.uint8)]
    logits = rng.standard_normal(151936).astype(np.float32)
    c = bfi_smp.PrefixCache(1 << 30, 0)
    s = torch.cuda.current_stream()
    toks = rng.integers(0, 151936, n).tolist()
    c.insert(toks, n, [_dev(t) for t in kv], [None, _dev(rec[1])], _dev(logits), stream=s.cuda_stream)
    s.synchronize()
    assert c.used_bytes() == n * 4 + logits.size * 4 + 4 * n * 8 * 128 * 2 + (1 << 20)
    hit = c.lookup(toks + [7, 8, 9])
    assert hit[1:] == (n, n)
    dst = [_dev(np.full_like(t, 0x5A5A)) for t in kv]
    rdst = [None, _dev(np.zeros(1 << 20, np.uint8))]
    ld = _dev(np.zeros_like(logits))
    got = c.restore(hit, dst, rdst, ld, stream=s.cuda_stream)
    s.synchronize()
    assert got == (n, True)
    for x, y in zip(dst, kv):
        x = x.cpu().numpy()
        assert np.array_equal(x[:n], y[:n]) and (x[n:] == 0).all()
    assert np.array_equal(rdst[1].cpu().numpy(), rec[1])
    assert np.array_equal(ld.cpu().numpy(), logits)
    c.close()


def test_device_cache_matches_the_oracle_on_random_sequences(gpu):
    rng = np.random.default_rng(11)
    for trial in range(3):
        budget = int(rng.integers(2_000, 40_000))
        dev, orc = DevCache(budget), OP.PrefixCache(budget)
        roots = [rng.integers(0, 4, int(rng.integers(1, 200))).tolist() for _ in range(4)]
        for step in range(60):
            root = roots[int(rng.integers(0, len(roots)))]
            ids = root[: int(rng.integers(0, len(root) + 1))] + rng.integers(0, 4, int(rng.integers(0, 80))).tolist()
            if rng.random() < 0.45:
                h1, h2 = dev.lookup(ids), orc.lookup(ids)
                assert (h1 is None) == (h2 is None)
                if h1 is None:
                    continue
                assert h1[1:] == h2[1:]
                like = kv_state(1) if orc.entries[h2[0]].rewindable else recurrent_state(1)
                got, want = dev.restore(h1, like), orc.restore(h2)
                assert got[0] == want[0] and (got[3] is None) == (want[3] is None)
                for x, y in zip(got[1], want[1]):
                    assert np.array_equal(x, y)
            elif ids:
                state = kv_state(min(len(ids), 512)) if rng.random() < 0.75 else recurrent_state(min(len(ids), 512))
                dev.insert(ids[: state[0]], state)
                n, kv, rec = state
                orc.insert(ids[: state[0]], n, kv, rec, LOGITS)
            assert len(dev) == len(orc) and dev.used_bytes() == orc.used
