"""GPU parity: the HIP sampler through the C ABI against the CPU oracle on the same seeded
inputs, bit for bit (tokens, kept sets, probabilities, the row maximum and the float32
normalizer; parity_util.compare_exact), at reduced and at full vocabulary."""
import numpy as np
import pytest

import bfi_smp
import oracle as O
import workloads
from parity_util import compare_exact

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def smp(gpu):
    s = bfi_smp.Sampler(0)
    yield s
    s.close()


def logits_f32(cfg):
    x = cfg["logits"]
    return workloads.bf16_bits_to_f32(x) if cfg["dtype"] == "bf16" else x


def run_gpu_target(smp, cfg, cap):
    import torch

    d = workloads.to_device(cfg)
    o = smp.target_rows(d["logits"], d["params"], d["u"], cap, d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in o.items()}


def run_oracle_target(cfg, cap):
    x = logits_f32(cfg)
    return O.target_rows(x, cfg["params"], cfg["hist"], cfg["hist_off"], cfg["u"], cfg["mask"], cap=cap,
                         want_s=True, threads=8)


def check(cfg, cap, smp):
    print(f"[parity] {cfg['name']} B={cfg['B']} V={cfg['V']} dtype={cfg['dtype']}", flush=True)
    g = run_gpu_target(smp, cfg, cap)
    o = run_oracle_target(cfg, cap)
    probs, stats = compare_exact(cfg, g, o)
    print(f"[parity] {cfg['name']}: {stats} problems={len(probs)}", flush=True)
    assert not probs, "\n".join(probs[:12])
    return g, o, stats


# ---- the reference's own known answers through the host-pointer entry point ----------


def S(smp, logits, prev, seed=0, mask=None, **params):
    return smp.sample_seeded(np.array(logits, np.float32), np.array(prev, np.uint32), params, seed, mask)


def test_reference_kats_on_gpu(smp):
    # sample.rs:466-689
    assert S(smp, [1.0, 0.0, 0.5], [], temperature=0.0) == 0
    assert S(smp, [0.1, 2.0, 1.5], [], temperature=0.0) == 1
    assert S(smp, [1.0, 0.0, 0.5], []) == 0
    m = bfi_smp.parse_id_union("root ::= id(1)", 3)
    assert S(smp, [9.0, 1.0, 8.0], [], temperature=0.0, mask=m) == 1
    assert S(smp, [1.2, 1.0], [0], temperature=0.0, repeat_penalty=1.5) == 1
    assert S(smp, [1.0, 0.5], [0], temperature=0.0, presence_penalty=0.5) == 0
    assert S(smp, [1.0, 100.0], [], temperature=10.0) <= 1
    assert S(smp, [1.0, 100.0], [], temperature=0.1) == 1
    assert S(smp, [10.0, 5.0, 2.0, 1.0], [], temperature=0.0, top_k=2) == 0
    for seed in range(32):
        assert S(smp, [10.0, 9.0, 8.0, 7.0], [], seed=seed, temperature=5.0, top_k=1) == 0
        assert S(smp, [10.0, 9.0, 8.0, 7.0], [], seed=seed, temperature=5.0, top_k=2) <= 1
    assert S(smp, [10.0, 5.0, 1.0, 0.1], [], temperature=1.0, top_p=0.5) == 0
    assert S(smp, [10.0, 5.0, 1.0, 0.1], [], temperature=1.0, top_p=0.999) <= 3
    assert S(smp, [], []) == 0  # empty logits -> Token(0)


def test_host_path_matches_oracle_on_random_small_rows(smp):
    rng = np.random.default_rng(7)
    bad = []
    for t in range(200):
        V = int(rng.integers(1, 300))
        x = (rng.standard_normal(V) * 3).astype(np.float32)
        prev = rng.integers(0, V + 3, int(rng.integers(0, 20))).astype(np.uint32)
        p = dict(temperature=float(rng.choice([0.0, 0.3, 1.0, 2.0])), top_k=int(rng.choice([0, 1, 5, 50, 400])),
                 top_p=float(rng.choice([1.0, 0.9, 0.5, 0.0])), min_p=float(rng.choice([0.0, 0.05, 0.5, 1.5])),
                 repeat_penalty=float(rng.choice([1.0, 1.3, 0.8])), presence_penalty=float(rng.choice([0.0, 0.7])),
                 frequency_penalty=float(rng.choice([0.0, 0.25])))
        mask = None
        if rng.random() < 0.3:
            mask = rng.integers(0, 2**32, (V + 31) // 32, dtype=np.uint64).astype(np.uint32)
        u = float(np.float32(rng.random()))
        g = smp.sample(x, prev, p, mask, u)
        o = O.sample(x, prev, p, mask, u)
        if g != o:
            bad.append((t, V, p, u, g, o))
    assert not bad, bad[:5]


# ---- the five configurations at reduced vocabulary ----------------------------------------


@pytest.mark.parametrize(
    "name,scale,greedy,seed",
    [
        ("C1", 0.1, False, 0),
        ("C1", 0.1, True, 0),
        ("C2", 0.05, False, 0),
        ("C2", 0.05, False, 1),
        ("C2", 0.05, True, 0),
        ("C3", 0.05, False, 0),
        ("C3", 0.05, True, 0),
        ("C5", 0.01, False, 0),
        ("C5", 0.1, False, 1),
    ],
)
def test_config_parity_reduced(smp, name, scale, greedy, seed):
    cfg = workloads.config(name, seed=seed, scale_v=scale, greedy=greedy)
    check(cfg, 2048, smp)


def test_c2_full_size_parity(smp):
    cfg = workloads.config("C2", seed=0)
    check(cfg, 2048, smp)


def test_c2_with_masks_full_size_parity(smp):
    """C2's rows under grammar allow-masks: penalties, top-k/top-p/min-p and a mask."""
    cfg = workloads.config("C2M", seed=0)
    check(cfg, 2048, smp)


def test_c3_full_size_parity(smp):
    """B=32 masked rows at V=151936, top-p 0.9 over whatever the mask allows (kept sets of
    thousands of ids)."""
    cfg = workloads.config("C3", seed=0)
    check(cfg, 8192, smp)


def test_c5_full_size_parity(smp):
    """B=256 rows of V=262144 bf16, top-p 0.9 over the full vocabulary (kept sets of about
    15,000 ids): every listed probability and the normalizer bit for bit."""
    cfg = workloads.config("C5", seed=0)
    check(cfg, 32768, smp)


def test_sample_rows_token_equals_target_token(smp):
    import torch

    cfg = workloads.config("C2", seed=2, scale_v=0.1)
    d = workloads.to_device(cfg)
    smp.sample_rows(d["logits"], d["params"], d["u"], d["out"], d["hist"], d["hist_off"], d["mask"])
    t = smp.target_rows(d["logits"], d["params"], d["u"], 0, d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    assert torch.equal(d["out"], t["token"])


# ---- spec verify ---------------------------------------------------------------------------


def oracle_verify(cfg, u_pairs=None, u_bonus=None):
    x = logits_f32(cfg)
    S, R = cfg["n_seq"], cfg["rows_per_seq"]
    up = cfg["u_pairs"] if u_pairs is None else u_pairs
    ub = cfg["u_bonus"] if u_bonus is None else u_bonus
    res = []
    for s in range(S):
        p = {k: (int(cfg["params"][s][k]) if k == "top_k" else float(cfg["params"][s][k]))
             for k in cfg["params"].dtype.names if k != "reserved"}
        dl = int(cfg["draft_len"][s])
        hist = cfg["hist"][cfg["hist_off"][s]:cfg["hist_off"][s + 1]]
        masks = None if cfg["mask"] is None else cfg["mask"][s * R: s * R + dl + 1]
        res.append(O.verify_seq(x[s * R: s * R + dl + 1], p, hist, cfg["drafts"][s, :dl], up[s, :dl].reshape(-1),
                                float(ub[s]), masks))
    return res


@pytest.mark.parametrize("greedy", [False, True])
def test_verify_parity(smp, greedy):
    import torch

    cfg = workloads.config("C4", seed=0, scale_v=0.05, greedy=greedy)
    # vary draft lengths, including 0
    cfg["draft_len"] = np.array([4, 3, 0, 1, 2, 4, 4, 4, 4, 4, 3, 4, 2, 4, 1, 4], np.int32)
    d = workloads.to_device(cfg)
    smp.verify(d["logits"], cfg["rows_per_seq"], d["params"], d["drafts"], d["draft_len"], d["u_pairs"],
               d["u_bonus"], d["out_accepted"], d["out_next"], d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    acc = d["out_accepted"].cpu().numpy()
    nxt = d["out_next"].cpu().numpy().astype(np.uint32)
    ref = oracle_verify(cfg)
    bad = [(s, int(acc[s]), int(nxt[s]), a_o, n_o) for s, (a_o, n_o) in enumerate(ref)
           if (acc[s], nxt[s]) != (a_o, n_o)]
    print(f"[parity] C4 greedy={greedy} accepted={acc.tolist()}", flush=True)
    assert not bad, bad


@pytest.mark.parametrize("greedy", [False, True])
def test_c4_full_size_verify_parity(smp, greedy):
    """16 sequences x (4 drafts + 1) rows at V=151936, T 0.8 / top-p 0.95 (and greedy): the
    accepted prefix length and the next token of every sequence equal the oracle's."""
    import torch

    cfg = workloads.config("C4", seed=0, greedy=greedy)
    d = workloads.to_device(cfg)
    smp.verify(d["logits"], cfg["rows_per_seq"], d["params"], d["drafts"], d["draft_len"], d["u_pairs"],
               d["u_bonus"], d["out_accepted"], d["out_next"], d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    acc = d["out_accepted"].cpu().numpy()
    nxt = d["out_next"].cpu().numpy().astype(np.uint32)
    ref = oracle_verify(cfg)
    bad = [(s, int(acc[s]), int(nxt[s]), a_o, n_o) for s, (a_o, n_o) in enumerate(ref)
           if (acc[s], nxt[s]) != (a_o, n_o)]
    print(f"[parity] C4 full greedy={greedy} accepted={acc.tolist()} next={nxt.tolist()}", flush=True)
    assert not bad, bad


# ---- edge cases ----------------------------------------------------------------------------


def _cfg_from(rows, params, hist=None, masks=None, u=None):
    x = np.array(rows, np.float32)
    B, V = x.shape
    if hist is None:
        hist = [[] for _ in range(B)]
    flat = np.array([t for h in hist for t in h], np.uint32)
    off = np.cumsum([0] + [len(h) for h in hist]).astype(np.int64)
    return dict(name="edge", B=B, V=V, dtype="f32", logits=x, params=bfi_smp.params_array(params), hist=flat,
                hist_off=off, mask=None if masks is None else np.array(masks, np.uint32),
                u=np.array(u if u is not None else [0.37] * B, np.float32))


def test_edge_cases(smp):
    rng = np.random.default_rng(3)
    V = 200
    base = (rng.standard_normal((1, V)) * 2).astype(np.float32)[0]
    W = (V + 31) // 32
    none_allowed = [0] * W
    one_allowed = [0] * W
    one_allowed[3] = 1 << 5
    cases = [
        (dict(temperature=1.0), None, None, 0.0),                         # u = 0, index order
        (dict(temperature=1.0, top_k=5), None, None, 0.0),                # u = 0, sorted
        (dict(temperature=0.8, min_p=2.0), [1, 2], None, 0.5),            # min-p fallback
        (dict(temperature=0.8, min_p=2.0, repeat_penalty=3.0), [int(np.argmax(base))], None, 0.5),
        (dict(temperature=1.0, top_k=V), None, None, 0.9),                # top-k >= V: inactive
        (dict(temperature=1.0, top_k=1), None, None, 0.9),
        (dict(temperature=1.0, top_p=0.0), None, None, 0.9),              # keeps exactly one
        (dict(temperature=1e-3, top_p=0.9), None, None, 0.9),
        (dict(temperature=1.0, repeat_penalty=1.5, presence_penalty=0.5, frequency_penalty=0.3),
         [5, 5, 5, 7, 1000, 7, 199], None, 0.42),                         # duplicates, id >= V
        (dict(temperature=1.0, top_p=0.9), None, none_allowed, 0.3),      # all masked, top-p only
        (dict(temperature=1.0, top_k=7), None, none_allowed, 0.3),        # all masked, top-k
        (dict(temperature=1.0, min_p=0.1), None, none_allowed, 0.3),      # all masked, min-p
        (dict(temperature=1.0), None, none_allowed, 0.3),                 # all masked, no filter
        (dict(temperature=0.0), None, none_allowed, 0.3),                 # all masked, greedy
        (dict(temperature=1.0, top_p=0.9), None, one_allowed, 0.3),       # exactly one allowed
        (dict(temperature=1.0, top_k=20), None, one_allowed, 0.3),        # fewer finite than k
        (dict(temperature=1.0, min_p=0.05), None, one_allowed, 0.99),
        (dict(temperature=1.0, top_p=0.999999), None, None, 0.999),
        (dict(temperature=0.0, repeat_penalty=0.5), [0, 1, 2], None, 0.1),  # rp < 1 raises penalized
    ]
    bad = []
    for i, (p, h, m, u) in enumerate(cases):
        cfg = _cfg_from([base], [p], [h or []], [m] if m is not None else None, [u])
        g = run_gpu_target(smp, cfg, 256)
        o = run_oracle_target(cfg, 256)
        probs, _ = compare_exact(cfg, g, o)
        if probs:
            bad.append((i, p, probs))
    assert not bad, bad


def test_ties_and_constant_rows(smp):
    V = 300
    rows = [np.zeros(V, np.float32), np.repeat(np.arange(30, dtype=np.float32), 10)]
    params = [dict(temperature=1.0, top_k=10), dict(temperature=1.0, top_p=0.5)]
    for r in rows:
        for p in params:
            cfg = _cfg_from([r], [p], u=[0.61])
            g = run_gpu_target(smp, cfg, 512)
            o = run_oracle_target(cfg, 512)
            probs, _ = compare_exact(cfg, g, o)
            assert not probs, (p, probs)


def test_unaligned_rows_and_odd_vocab(smp):
    import torch

    for V in (1, 7, 33, 4099, 8193):
        cfg = workloads.config("C2", seed=5, scale_v=1.0)
        x = cfg["logits"][:8, :V].copy()
        sub = dict(cfg)
        sub.update(B=8, V=V, logits=x, params=cfg["params"][:8], u=cfg["u"][:8])
        h = [cfg["hist"][cfg["hist_off"][b]:cfg["hist_off"][b + 1]] % V for b in range(8)]
        sub["hist"] = np.concatenate(h).astype(np.uint32)
        sub["hist_off"] = cfg["hist_off"][:9]
        check(sub, 256, smp)
    # a row stride larger than V with an unaligned base: the scalar-load path
    cfg = workloads.config("C2", seed=6, scale_v=0.02)
    d = workloads.to_device(cfg)
    big = torch.zeros((cfg["B"], cfg["V"] + 3), dtype=torch.float32, device="cuda")
    big[:, 1:cfg["V"] + 1] = d["logits"]
    view = big[:, 1:cfg["V"] + 1]
    smp.sample_rows(view, d["params"], d["u"], d["out"], d["hist"], d["hist_off"], d["mask"])
    ref = torch.zeros_like(d["out"])
    smp.sample_rows(d["logits"], d["params"], d["u"], ref, d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    assert torch.equal(d["out"], ref)


def test_repeated_launches_are_deterministic(smp):
    import torch

    cfg = workloads.config("C2", seed=9, scale_v=0.1)
    d = workloads.to_device(cfg)
    outs = []
    for _ in range(5):
        smp.sample_rows(d["logits"], d["params"], d["u"], d["out"], d["hist"], d["hist_off"], d["mask"])
        outs.append(d["out"].clone())
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


# ---- history corrections, fallback paths, magnitudes ---------------------------------------

MODES = [
    dict(temperature=0.0),
    dict(temperature=0.9, top_k=50),
    dict(temperature=0.9, top_p=0.9),
    dict(temperature=0.9, min_p=0.05),
    dict(temperature=0.9),
    dict(temperature=0.9, min_p=0.05, top_p=0.95),
    dict(temperature=0.9, top_k=20, top_p=0.8, min_p=0.02),
]
PENALTIES = [
    dict(repeat_penalty=1.5),
    dict(repeat_penalty=0.7),
    dict(presence_penalty=-0.8, frequency_penalty=0.2),
    dict(repeat_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.4),
]


def test_history_holds_chunk_maxima(smp):
    """Histories made of each row's largest logits: most chunks' maxima are penalized, so the
    select pass re-derives those chunks' statistics."""
    rng = np.random.default_rng(11)
    V = 50000
    params, hist, rows = [], [], []
    for m in MODES:
        for p in PENALTIES:
            x = (rng.standard_normal(V) * 2).astype(np.float32)
            top = np.argsort(-x, kind="stable")[:300]
            h = np.concatenate([top, top[:40], top[:10]]).astype(np.uint32)  # repeats for counts
            rng.shuffle(h)
            rows.append(x)
            hist.append(h.tolist())
            params.append({**m, **p})
    u = rng.random(len(rows)).astype(np.float32)
    cfg = _cfg_from(rows, params, hist, u=u.tolist())
    cfg["name"] = "dirty-chunks"
    check(cfg, 512, smp)


def test_history_larger_than_the_hash(smp):
    """More distinct history ids than the select pass's LDS hash holds: whole-row passes."""
    rng = np.random.default_rng(12)
    V = 30000
    params, hist, rows = [], [], []
    for m in MODES:
        x = (rng.standard_normal(V) * 2).astype(np.float32)
        ids = rng.choice(V, 3000, replace=False)
        h = np.concatenate([ids, ids[:700], np.argsort(-x)[:20]]).astype(np.uint32)
        rows.append(x)
        hist.append(h.tolist())
        params.append({**m, "repeat_penalty": 1.2, "presence_penalty": 0.3, "frequency_penalty": 0.1})
    u = rng.random(len(rows)).astype(np.float32)
    cfg = _cfg_from(rows, params, hist, u=u.tolist())
    cfg["name"] = "large-history"
    check(cfg, 512, smp)


def test_min_p_only_rows_beyond_the_candidate_lists(smp):
    """Flat rows under min-p alone keep most of the vocabulary, in index order."""
    rng = np.random.default_rng(13)
    V = 75968
    rows = [(rng.standard_normal(V) * 0.05).astype(np.float32) for _ in range(4)]
    params = [dict(temperature=1.0, min_p=0.05), dict(temperature=0.5, min_p=0.9),
              dict(temperature=1.0, min_p=0.05, repeat_penalty=1.3), dict(temperature=2.0, min_p=0.5)]
    hist = [[], [], rng.choice(V, 500, replace=False).tolist(), []]
    cfg = _cfg_from(rows, params, hist, u=[0.0, 0.5, 0.77, 0.999])
    cfg["name"] = "min-p-flat"
    check(cfg, 256, smp)


def test_extreme_magnitudes(smp):
    """Logits outside [2^-100, 2^100) take IEEE division; the values must match it exactly."""
    rng = np.random.default_rng(14)
    V = 20000
    rows = []
    for k in range(4):
        x = rng.standard_normal(V).astype(np.float32)
        x[rng.choice(V, 50, replace=False)] = np.float32(1e-35)
        x[rng.choice(V, 50, replace=False)] = np.float32(-3e-39)
        if k % 2:
            x[rng.choice(V, 3, replace=False)] = np.float32(2.0 ** 110)
            x[rng.choice(V, 3, replace=False)] = np.float32(-(2.0 ** 120))
        rows.append(x)
    params = [dict(temperature=0.7, top_k=40), dict(temperature=0.7, top_p=0.9), dict(temperature=1.3),
              dict(temperature=0.7, min_p=0.1)]
    cfg = _cfg_from(rows, params, u=[0.3, 0.6, 0.9, 0.1])
    cfg["name"] = "magnitudes"
    check(cfg, 256, smp)


def _restreams(smp, cfg, cap):
    """Per row: ranges the row kernel streamed exactly in a traced call (the phase trace keeps
    the quantizing pass's workgroups' words (8 each), then 16 per row, word 9 that count)."""
    import torch

    d = workloads.to_device(cfg)
    smp.set_tracing(True)
    smp.target_rows(d["logits"], d["params"], d["u"], cap, d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    smp.set_tracing(False)
    tr = smp.trace().astype(np.int64)
    B = cfg["B"]
    nrc = (tr.size - B * 16) // 16
    return tr[nrc * 8:nrc * 8 + B * 16].reshape(B, 16)[:, 9]


def test_rows_whose_sum_outruns_the_prediction(smp):
    """The reference's f32 normalizer drops every term below half a unit of its running sum.
    Rows whose two large terms bring the sum just below 2, then ~150K terms each below half a
    unit: the exact prefix the quantizing pass predicts from passes 2 while
    the reference's sum stays below it, so the chain's binade checks fail (and chunks straddling
    the boundary list more windows than they may) and the row kernel streams those chunks
    exactly. The lost mass (~0.0087) exceeds the prediction's margin at 2 for the last chunks.
    Tokens and kept sets must still be the reference's, and the exact streams must have run."""
    rng = np.random.default_rng(17)
    V = 151936
    modes = [dict(temperature=1.0, top_p=0.9), dict(temperature=1.0), dict(temperature=1.0, min_p=0.3),
             dict(temperature=1.0, top_k=3)]
    rows, params = [], []
    for k, m in enumerate(modes):
        x = (-16.68 + rng.standard_normal(V) * 0.005).astype(np.float32)
        x[0] = 0.0
        x[1] = np.float32(np.log(0.996 - 0.0005 * k))
        rows.append(x)
        params.append(m)
    # the premise: every small term is below half a unit of [1, 2), and the exact sum passes 2
    e = np.exp(np.array(rows, np.float64))
    assert e[:, 2:].max() < 2.0 ** -24 and (e.sum(1) > 2.0).all() and (e[:, :2].sum(1) < 2.0).all()
    cfg = _cfg_from(rows, params, u=[0.2, 0.999, 0.5, 0.7])
    cfg["name"] = "outrun"
    check(cfg, 512, smp)
    assert (_restreams(smp, cfg, 512) > 0).all()


def test_c1_full_size_and_topk_over_many_chunks(smp):
    """B=1 at full vocabulary: 75 chunks each hand over their own top-k, so the list above
    the largest chunk bound holds thousands of entries and the select narrows it to about k."""
    cfg = workloads.config("C1", seed=0)
    check(cfg, 2048, smp)
    rng = np.random.default_rng(15)
    V = 151936
    rows = [(rng.standard_normal(V) * 2.5).astype(np.float32) for _ in range(4)]
    params = [dict(temperature=0.7, top_k=40, top_p=0.95), dict(temperature=1.2, top_k=200),
              dict(temperature=1.0, top_k=1000, top_p=0.99), dict(temperature=0.9, top_k=40, min_p=0.01)]
    hist = [rng.integers(0, V, 64).tolist(), [], rng.integers(0, V, 300).tolist(), []]
    for i in range(4):
        params[i]["repeat_penalty"] = 1.1 if hist[i] else 1.0
        cfg = _cfg_from([rows[i]], [params[i]], [hist[i]], u=[0.3 + 0.2 * i])
        cfg["name"] = f"topk-many-chunks-{i}"
        check(cfg, 2048, smp)


def test_topk_bound_from_chunk_maxima(smp):
    """Single rows over 75 chunks with top-k <= chunks, where the k-th largest chunk maximum
    bounds the list: values on a coarse grid (exact ties in s, and so in p, at the bound,
    kept in index order), a row whose other values lie more than 64 below the maximum (p
    underflows: the bound stays off and zero-probability elements fill the top-k in index
    order), a mask that leaves fewer than k chunks with an allowed element, and a history
    that penalizes chunk maxima."""
    rng = np.random.default_rng(21)
    V = 151936
    W = (V + 31) // 32
    grid = (np.round(rng.standard_normal(V) * 10.0) / 4.0).astype(np.float32)
    far = (rng.standard_normal(V)).astype(np.float32)
    far[777] = np.float32(150.0)
    sparse = (rng.standard_normal(V) * 2.5).astype(np.float32)
    mask = np.zeros(W, np.uint32)
    for w in rng.choice(W, 6, replace=False):  # at most 6 chunks hold allowed ids
        mask[w] = np.uint32(0xFFFFFFFF)
    pen = (rng.standard_normal(V) * 2.5).astype(np.float32)
    chunk = 2048
    maxima = [int(c * chunk + np.argmax(pen[c * chunk:(c + 1) * chunk])) for c in range(V // chunk)]
    cases = [
        ("grid-k40", grid, dict(temperature=1.0, top_k=40), None, None, 0.61),
        ("grid-k75-topp", grid, dict(temperature=0.5, top_k=75, top_p=0.9), None, None, 0.13),
        ("far-k40", far, dict(temperature=1.0, top_k=40), None, None, 0.999),
        ("far-k8-t03", far, dict(temperature=0.3, top_k=8), None, None, 0.5),
        ("masked-k20", sparse, dict(temperature=1.0, top_k=20), None, mask, 0.77),
        ("pen-k30", pen, dict(temperature=0.8, top_k=30, repeat_penalty=1.3), maxima[:40], None, 0.4),
    ]
    for name, x, prm, hist, m, u in cases:
        cfg = _cfg_from([x], [prm], [hist or []], None if m is None else [m], u=[u])
        cfg["name"] = f"topk-chunk-maxima-{name}"
        check(cfg, 2048, smp)


def test_verify_with_penalties(smp):
    """Spec verify with histories and penalties: row i of a sequence also counts the drafts
    before it (spec.rs:137-162 appends each accepted draft), both for histories the stream
    pass applies and for longer ones the row pass applies itself."""
    import torch

    rng = np.random.default_rng(16)
    cfg = workloads.config("C4", seed=1, scale_v=0.25)
    S, R, V = cfg["n_seq"], cfg["rows_per_seq"], cfg["V"]
    hists = []
    for s in range(S):
        n = [0, 40, 700, 1500][s % 4]
        h = rng.integers(0, V, n).astype(np.uint32)
        if n:
            h[: min(n, 8)] = cfg["drafts"][s, 0]  # the first draft repeated: counts > 1
        hists.append(h)
    cfg["hist"] = np.concatenate(hists).astype(np.uint32) if any(len(h) for h in hists) else np.zeros(0, np.uint32)
    cfg["hist_off"] = np.cumsum([0] + [len(h) for h in hists]).astype(np.int64)
    params = cfg["params"].copy()
    for s in range(S):
        params[s]["repeat_penalty"] = [1.0, 1.3, 0.8, 1.1][s % 4]
        params[s]["presence_penalty"] = [0.0, 0.4, -0.2, 0.5][(s // 4) % 4]
        params[s]["frequency_penalty"] = [0.0, 0.2][s % 2]
        params[s]["top_k"] = [40, 100, 20, 60][(s // 2) % 4]
        params[s]["min_p"] = [0.0, 0.05][(s // 8) % 2]
    cfg["params"] = params
    d = workloads.to_device(cfg)
    smp.verify(d["logits"], R, d["params"], d["drafts"], d["draft_len"], d["u_pairs"], d["u_bonus"],
               d["out_accepted"], d["out_next"], d["hist"], d["hist_off"], d["mask"])
    torch.cuda.synchronize()
    acc = d["out_accepted"].cpu().numpy()
    nxt = d["out_next"].cpu().numpy().astype(np.uint32)
    ref = oracle_verify(cfg)
    bad = [(s, int(acc[s]), int(nxt[s]), a_o, n_o) for s, (a_o, n_o) in enumerate(ref)
           if (acc[s], nxt[s]) != (a_o, n_o)]
    print(f"[parity] verify+penalties accepted={acc.tolist()}", flush=True)
    assert not bad, bad


def test_penalized_rows_across_chunks(smp):
    """Penalties over many chunks: greedy rows (argmax of the penalized logits), rows with
    min_p > 1 (fallback to the masked, un-penalized argmax, which a penalty may have moved),
    top-k / top-p / min-p rows; histories just below and above the stream pass's limit, with
    duplicates, ids >= V and the row maximum in them."""
    rng = np.random.default_rng(17)
    V = 60000
    rows, params, hist = [], [], []
    modes = [dict(temperature=0.0), dict(temperature=0.9, min_p=2.0), dict(temperature=0.9, top_k=30),
             dict(temperature=1.1, top_p=0.9, min_p=0.02), dict(temperature=0.6, min_p=0.1)]
    for m in modes:
        for n in (1024, 1025, 300):
            x = (rng.standard_normal(V) * 2.0).astype(np.float32)
            x[rng.choice(V, 6, replace=False)] += 8.0
            h = rng.integers(0, V, n).astype(np.uint32)
            h[:5] = np.argmax(x)  # the row maximum, five times
            h[5] = V + 7  # outside the vocabulary: ignored
            rows.append(x)
            hist.append(h.tolist())
            params.append({**m, "repeat_penalty": 1.4, "presence_penalty": 0.3, "frequency_penalty": 0.25})
    u = rng.random(len(rows)).astype(np.float32)
    cfg = _cfg_from(rows, params, hist, u=u.tolist())
    cfg["name"] = "penalized-rows"
    check(cfg, 512, smp)
