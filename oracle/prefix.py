"""CPU restatement of the reference's prefix cache (crates/bfi-runtime/src/engine/prefix.rs),
test infrastructure only: the checker of the library's bfi_pc_* entry points, never called by
the product path.

Entries hold their state as numpy arrays (the kept K/V rows, recurrent tensors, logits). The
reference's rolling hash only selects probe candidates that it then confirms token by token, so
this restatement keys its marks by the token prefix itself (a collision-free hash); the probe
order, the confirmation, the rewind rules, the byte accounting and the eviction order follow
prefix.rs line by line.

Pins: the reference's own unit tests (prefix.rs:392-498) are restated as known-answer tests in
tests/test_prefix_cpu.py and run against this module and the library; the library is compared
with this module on random operation sequences there too.
"""
from __future__ import annotations

import numpy as np

BLOCK = 64  # prefix.rs:29


class Entry:
    def __init__(self, tokens, kv, rec, logits, rewindable, nbytes, last_used, marks):
        self.tokens = tokens
        self.kv = kv          # [(kind, array)], kind "rows" (kept rows, full row count) or "whole"
        self.rec = rec        # [array or None]
        self.logits = logits
        self.rewindable = rewindable
        self.bytes = nbytes
        self.last_used = last_used
        self.marks = marks


class PrefixCache:
    """prefix.rs:114-347."""

    def __init__(self, budget_bytes: int):  # prefix.rs:132-142
        self.entries: dict[int, Entry] = {}
        self.marks: dict[tuple, list[int]] = {}
        self.budget = budget_bytes
        self.used = 0
        self.next_id = 0
        self.tick = 0
        self.forwarded = 0

    def __len__(self):
        return len(self.entries)

    def note_forward(self, n):  # prefix.rs:148-150
        self.forwarded += n

    def lookup(self, ids):  # prefix.rs:168-214
        ids = list(ids)
        probes = []
        for i in range(len(ids)):
            for eid in self.marks.get(tuple(ids[:i + 1]), []):
                probes.append((i + 1, eid))
        best = None
        for length, eid in reversed(probes):
            if best is not None and best[0] >= length + BLOCK:
                break
            e = self.entries.get(eid)
            if e is None:
                continue
            if len(e.tokens) < length or e.tokens[:length] != ids[:length]:
                continue
            if e.rewindable:
                matched = length + _common(e.tokens[length:], ids[length:])
            elif length == len(e.tokens):
                matched = length
            else:
                continue
            if best is None or matched > best[0]:
                best = (matched, eid)
        if best is None or best[0] < BLOCK:
            # (equal shares found here go to the oldest entry: the reference iterates a hash
            # map, whose order it leaves open; this dict iterates in insertion order)
            for eid, e in self.entries.items():
                if not e.rewindable:
                    continue
                m = _common(e.tokens, ids)
                if m > 0 and (best is None or m > best[0]):
                    best = (m, eid)
        if best is None:
            return None
        matched, eid = best
        e = self.entries[eid]
        restore = matched if matched == len(e.tokens) else min(matched, max(len(ids) - 1, 0))
        return (eid, matched, restore) if restore > 0 else None

    def restore(self, hit):  # prefix.rs:217-230
        eid, matched, restore = hit
        self.tick += 1
        e = self.entries.get(eid)
        if e is None:
            return None
        e.last_used = self.tick
        kv = []
        for kind, arr, full_rows in e.kv:
            if kind == "rows":
                out = np.zeros((full_rows,) + arr.shape[1:], arr.dtype)
                out[:arr.shape[0]] = arr
                kv.append(out)
            else:
                kv.append(arr.copy())
        rec = [None if r is None else r.copy() for r in e.rec]
        logits = e.logits.copy() if restore == len(e.tokens) else None
        return restore, kv, rec, logits

    def insert(self, tokens, n, kv, rec, logits, whole=()):  # prefix.rs:233-260
        tokens = list(tokens)
        if not tokens or n != len(tokens):
            return
        kept = []
        for i, t in enumerate(kv):
            if i in whole:
                kept.append(("whole", t.copy(), None))
            else:
                kept.append(("rows", t[:min(n, t.shape[0])].copy(), t.shape[0]))
        self._insert_entry(tokens, kept, [None if r is None else r.copy() for r in rec], logits.copy())

    def _insert_entry(self, tokens, kv, rec, logits):  # prefix.rs:262-307
        rewindable = all(r is None for r in rec)
        nbytes = (len(tokens) * 4 + logits.size * 4 + sum(a.nbytes for _, a, _ in kv)
                  + sum(r.nbytes for r in rec if r is not None))
        if nbytes > self.budget:
            return
        self._drop_superseded(tokens, rewindable)
        while self.used + nbytes > self.budget:
            if not self._evict_lru():
                break
        marks = []
        for i in range(len(tokens)):
            length = i + 1
            if length == len(tokens) or (rewindable and length % BLOCK == 0):
                marks.append(tuple(tokens[:length]))
        self.tick += 1
        eid = self.next_id
        self.next_id += 1
        for m in marks:
            self.marks.setdefault(m, []).append(eid)
        self.used += nbytes
        self.entries[eid] = Entry(tokens, kv, rec, logits, rewindable, nbytes, self.tick, marks)

    def _drop_superseded(self, tokens, rewindable):  # prefix.rs:310-322
        doomed = [eid for eid, e in self.entries.items()
                  if e.tokens == tokens or (rewindable and e.rewindable and tokens[:len(e.tokens)] == e.tokens)]
        for eid in doomed:
            self._remove(eid)

    def _evict_lru(self):  # prefix.rs:324-333
        if not self.entries:
            return False
        self._remove(min(self.entries, key=lambda k: self.entries[k].last_used))
        return True

    def _remove(self, eid):  # prefix.rs:335-347
        e = self.entries.pop(eid, None)
        if e is None:
            return
        self.used -= e.bytes
        for m in e.marks:
            lst = self.marks.get(m)
            if lst is None:
                continue
            lst[:] = [x for x in lst if x != eid]
            if not lst:
                del self.marks[m]


def _common(a, b):  # prefix.rs:356-358
    n = 0
    for x, y in zip(a, b):
        if x != y:
            break
        n += 1
    return n
