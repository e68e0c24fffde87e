"""Pins of the CPU oracle beyond the reference's own known-answer tests.

The oracle is a restatement; these checks use mechanics of their own so that a plausible
mistake in it (a dropped term, a swapped step, a wrong comparison, an unstable tie order)
fails at least one of them:
  - brute force in float64 with Python's sorted() over every parameter combination at
    V <= 8, on logits and penalties that are exact in binary (so f32 vs f64 rounding cannot
    decide an outcome), comparing tokens away from CDF boundaries and kept sets away from
    top-p boundaries;
  - numpy closed forms at V in the thousands: IEEE f32 penalties/division (numpy's own f32
    ops), f64 softmax, top-k by np.argsort(kind="stable"), top-p by f64 cumsum, min-p;
  - exact edge cases (cum == top_p, u == p_d/sum, u == 0, ties).
test_pins_catch_planted_mistakes rebuilds the oracle with each ORC_MUTATE mistake and checks
that these pins reject every one of them.
"""
import itertools
import math
import os
import subprocess
import tempfile

import numpy as np
import pytest

import oracle as O

ORACLE_DIR = os.path.dirname(O.__file__)


# ---- f64 brute force (Python sorted(), sets) ---------------------------------------------


def bf_target(logits, prev, p, mask=None):
    V = len(logits)
    x = [(-math.inf if (mask is not None and not ((int(mask[i >> 5]) >> (i & 31)) & 1)) else float(l))
         for i, l in enumerate(logits)]
    masked = list(x)
    seen = set(int(t) for t in prev if int(t) < V)
    cnt = {t: sum(1 for q in prev if int(q) == t) for t in seen}
    rp, pp, fp = p.get("repeat_penalty", 1.0), p.get("presence_penalty", 0.0), p.get("frequency_penalty", 0.0)
    if abs(rp - 1.0) > 1.1920929e-07 and len(prev):
        for t in seen:
            x[t] = x[t] / rp if x[t] > 0 else x[t] * rp
    if pp != 0 and len(prev):
        for t in seen:
            x[t] -= pp
    if fp != 0 and len(prev):
        for t in seen:
            x[t] -= fp * cnt[t]
    T = p.get("temperature", 0.0)
    if not T > 0:
        best = max(range(V), key=lambda i: (x[i], -i)) if V else 0
        return ("token", best if x[best] > -math.inf else 0), None
    s = [v / T for v in x]
    M = max(s)
    e = [math.exp(v - M) for v in s]
    Z = sum(e)
    pr = [v / Z for v in e]
    k, top_p, min_p = p.get("top_k", 0), p.get("top_p", 1.0), p.get("min_p", 0.0)
    order = list(range(V))
    sort = (0 < k < V) or top_p < 1.0
    if sort:
        order = sorted(order, key=lambda i: (-pr[i], i))
    bands = []
    if 0 < k < V:
        order = order[:k]
    if top_p < 1.0:
        c, cut = 0.0, len(order)
        for j, i in enumerate(order):
            c += pr[i]
            bands.append(c)
            if c >= top_p:
                cut = j + 1
                break
        order = order[: max(cut, 1)]
    if min_p > 0:
        th = min_p * max(pr[i] for i in order)
        order = [i for i in order if pr[i] >= th]
        if not order:
            best = max(range(V), key=lambda i: (masked[i], -i))
            return ("token", best if masked[best] > -math.inf else 0), None
    return ("weights", [(i, pr[i]) for i in order]), dict(bands=bands, top_p=top_p, pr=pr)


def bf_draw(w, u):
    tot = sum(b for _, b in w)
    r = u * tot
    c = 0.0
    for i, b in w:
        c += b
        if r <= c:
            return i
    return w[-1][0]


def cdf_boundary_dist(w, u):
    tot = sum(b for _, b in w)
    c, d = 0.0, abs(u)
    for _, b in w:
        c += b
        d = min(d, abs(u - c / tot))
    return d


def _tiny_cases():
    rng = np.random.default_rng(1234)
    grid = np.arange(-16, 17) / 8.0  # exact in binary
    for V in (1, 2, 3, 5, 8):
        for rep in range(6):
            logits = rng.choice(grid, V).astype(np.float32)
            if rep == 0 and V > 1:
                logits[:] = logits[0]  # all tied
            prev = rng.integers(0, V + 2, rng.integers(0, 4)).astype(np.uint32)
            mask = None
            if rep % 3 == 2:
                allowed = rng.random(V) < 0.6
                allowed[rng.integers(0, V)] = True
                mask = np.zeros(1, np.uint32)
                for i in np.nonzero(allowed)[0]:
                    mask[0] |= np.uint32(1 << int(i))
            yield V, logits, prev, mask


PARAM_GRID = dict(
    temperature=[0.0, 0.5, 1.0, 2.0],
    top_k=[0, 1, 2, 3, 9],
    top_p=[1.0, 0.5, 0.75, 0.9],
    min_p=[0.0, 0.25, 0.5],
    pen=[(1.0, 0.0, 0.0), (2.0, 0.0, 0.0), (0.5, 0.5, 0.0), (2.0, 1.0, 0.125), (1.0, -0.25, 0.25)],
)
U_GRID = [0.0, 0.1, 0.3, 0.5, 0.7, 0.9, 0.999]


def check_bruteforce(fail):
    n = 0
    for V, logits, prev, mask in _tiny_cases():
        for T, k, tp, mp, (rp, pp, fp) in itertools.product(*PARAM_GRID.values()):
            p = dict(temperature=T, top_k=k, top_p=tp, min_p=mp, repeat_penalty=rp, presence_penalty=pp,
                     frequency_penalty=fp)
            ref, aux = bf_target(logits, prev, p, mask)
            got = O.target(logits, prev, p, mask, want_s=True)
            n += 1
            if ref[0] == "token":
                if got["kind"] != 0 or got["token"] != ref[1]:
                    fail(f"token target V={V} p={p} ref={ref} got={got['kind'], got['token']}")
                continue
            if got["kind"] != 1:
                fail(f"kind V={V} p={p}")
                continue
            near_band = aux["bands"] and any(abs(b - aux["top_p"]) < 1e-5 for b in aux["bands"])
            ids_ref = [i for i, _ in ref[1]]
            if not near_band:
                if list(got["ids"]) != ids_ref:
                    fail(f"kept V={V} p={p} ref={ids_ref} got={list(got['ids'])}")
                    continue
                for (i, pr), g in zip(ref[1], got["w"]):
                    if abs(g - pr) > 1e-5 * max(pr, 1e-30) + 1e-37:
                        fail(f"prob V={V} p={p} id={i} {g} vs {pr}")
            for u in U_GRID:
                if near_band or cdf_boundary_dist(ref[1], u) < 1e-5:
                    continue
                t = O.sample(logits, prev, p, mask, u)
                if t != bf_draw(ref[1], u):
                    fail(f"draw V={V} p={p} u={u}: {t} vs {bf_draw(ref[1], u)}")
    return n


# ---- numpy closed forms at larger V ------------------------------------------------------


def check_closed_forms(fail):
    rng = np.random.default_rng(99)
    for V in (257, 1000, 4096):
        for trial in range(4):
            logits = (rng.standard_normal(V) * 2.5).astype(np.float32)
            logits[rng.integers(0, V, 4)] += 8
            prev = rng.integers(0, V, 40).astype(np.uint32)
            rp, pp, fp = np.float32(1.3), np.float32(0.4), np.float32(0.2)
            T = np.float32([0.7, 1.0, 1.3, 0.35][trial])
            mask = None
            if trial == 3:
                mask = rng.integers(0, 2**32, (V + 31) // 32, dtype=np.uint64).astype(np.uint32)
            p = dict(temperature=float(T), repeat_penalty=float(rp), presence_penalty=float(pp),
                     frequency_penalty=float(fp))
            got = O.target(logits, prev, p, mask, want_s=True)
            # IEEE f32 penalties and division, computed with numpy's own f32 ops
            x = logits.copy()
            if mask is not None:
                allowed = ((mask[np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1).astype(bool)
                x[~allowed] = -np.inf
            ids, counts = np.unique(prev, return_counts=True)
            for i, c in zip(ids, counts):
                v = x[i]
                v = v / rp if v > 0 else v * rp
                v = np.float32(v - pp)
                v = np.float32(v - np.float32(fp * np.float32(c)))
                x[i] = v
            s = (x / T).astype(np.float32)
            if not np.array_equal(got["s"].view(np.uint32), s.view(np.uint32)):
                fail(f"penalty/temperature closed form V={V} trial={trial}")
            # softmax over the full V in f64
            pr = np.exp(s.astype(np.float64) - s.max())
            pr /= pr.sum()
            if not np.allclose(got["w"], pr, rtol=2e-5, atol=1e-30):
                fail(f"softmax closed form V={V} trial={trial}")
            # top-k via np.argsort (stable)
            k = [5, 50, 100, 1][trial]
            q = dict(p, top_k=k)
            g = O.target(logits, prev, q, mask)
            want = np.argsort(-pr, kind="stable")[:k]
            if list(g["ids"]) != list(want):
                fail(f"top-k argsort V={V} k={k}")
            # top-p via f64 cumsum
            tp = [0.9, 0.5, 0.95, 0.8][trial]
            q = dict(p, top_p=tp)
            g = O.target(logits, prev, q, mask)
            order = np.argsort(-pr, kind="stable")
            cum = np.cumsum(pr[order])
            cut = int(np.searchsorted(cum, tp) + 1)
            near = np.min(np.abs(cum - tp)) < 1e-5
            if not near and list(g["ids"]) != list(order[:cut]):
                fail(f"top-p cumsum V={V} p={tp}: {len(g['ids'])} vs {cut}")
            # min-p (index order kept, threshold min_p * max p)
            mp = 0.05
            q = dict(p, min_p=mp)
            g = O.target(logits, prev, q, mask)
            keep = np.nonzero(pr >= mp * pr.max() * (1 + 1e-6))[0]
            edge = np.nonzero(np.abs(pr - mp * pr.max()) <= 1e-6 * pr.max())[0]
            if not set(keep) <= set(g["ids"]) or not set(g["ids"]) <= set(keep) | set(edge):
                fail(f"min-p V={V}")
            if list(g["ids"]) != sorted(g["ids"]):
                fail(f"min-p keeps index order V={V}")


# ---- exact edge cases --------------------------------------------------------------------


def check_edges(fail):
    # cum == top_p exactly: p = [0.5, 0.5], top_p 0.5 keeps one (first cum >= p)
    g = O.target(np.zeros(2, np.float32), [], dict(temperature=1.0, top_p=0.5))
    if g["len"] != 1 or list(g["ids"]) != [0]:
        fail("top-p cum == p keeps 1")
    # u == p_d / sum exactly: strict u < p_d/sum rejects (spec.rs:86)
    if O.judge(("weights", [(1, 0.5), (2, 0.5)]), 1, 0.5, 0.0) != ("reject", 2):
        fail("judge strict u < p_d/sum")
    # u == 0 draws the first element even with zero weight (r <= cum inclusive)
    if O.draw([5, 6, 7], [0.0, 0.5, 0.5], 0.0) != 5:
        fail("draw r <= cum inclusive at u=0")
    # greedy tie -> lowest index
    if O.sample(np.ones(4, np.float32), [], dict(temperature=0.0)) != 0:
        fail("argmax tie lowest index")
    # repeat then presence: [2, 0.25], prev [0], rp 2, pp 1 -> s0 = 2/2 - 1 = 0 < 0.25
    if O.sample(np.array([2.0, 0.25], np.float32), [0], dict(repeat_penalty=2.0, presence_penalty=1.0)) != 1:
        fail("penalty order repeat -> presence")
    # repeat multiplies non-positive logits: [-1, -1.5], prev [0], rp 2 -> s0 = -2 < -1.5
    if O.sample(np.array([-1.0, -1.5], np.float32), [0], dict(repeat_penalty=2.0)) != 1:
        fail("repeat multiplies negatives")
    # min-p > 1 empties vals -> argmax of masked, un-penalized logits (sample.rs:415-422)
    g = O.target(np.array([2.0, 1.9], np.float32), [0], dict(temperature=1.0, min_p=2.0, repeat_penalty=2.0),
                 want_s=True)
    if g["kind"] != 0 or g["token"] != 0:
        fail("min-p fallback uses masked un-penalized logits")
    # stable ties under top-k: equal logits keep index order
    g = O.target(np.ones(6, np.float32), [], dict(temperature=1.0, top_k=3))
    if list(g["ids"]) != [0, 1, 2]:
        fail("stable tie order under top-k")
    # a draft must come from the most recent n-gram match
    if O.draft([1, 2, 10, 11, 1, 2, 20, 21, 7, 1, 2], 2, 3, 2) != [20, 21]:
        fail("draft most recent")
    # judge residual excludes d
    if O.judge(("weights", [(1, 0.75), (2, 0.25)]), 1, 0.9, 0.3) != ("reject", 2):
        fail("judge residual excludes d")


def _run_all():
    failures = []
    check_edges(failures.append)
    check_closed_forms(failures.append)
    n = check_bruteforce(failures.append)
    return failures, n


def test_oracle_edges():
    f = []
    check_edges(f.append)
    assert not f, f


def test_oracle_closed_forms():
    f = []
    check_closed_forms(f.append)
    assert not f, f[:10]


def test_oracle_bruteforce_tiny_vocab():
    f = []
    n = check_bruteforce(f.append)
    assert n > 10000
    assert not f, f[:10]


MUTANTS = list(range(1, 14))


def test_pins_catch_planted_mistakes():
    src = os.path.join(ORACLE_DIR, "bfi_oracle.c")
    with tempfile.TemporaryDirectory() as td:
        caught = {}
        for m in MUTANTS:
            so = os.path.join(td, f"mut{m}.so")
            subprocess.run(
                ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", f"-DORC_MUTATE={m}",
                 "-o", so, src, "-lm", "-lpthread"],
                check=True,
            )
            prev = O.use_library(so)
            try:
                f = []
                check_edges(f.append)
                if not f:
                    check_closed_forms(f.append)
                if not f:
                    check_bruteforce(f.append)
                caught[m] = bool(f)
            finally:
                O.restore_library(prev)
        missed = [m for m, c in caught.items() if not c]
        assert not missed, f"planted mistakes not caught: {missed}"
