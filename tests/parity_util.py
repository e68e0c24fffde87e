"""Comparison of GPU results with the CPU oracle under the parity bar of the sampling path.

Token ids must equal the oracle's. The only exemption is a draw whose u lies within 1e-6
of a CDF boundary, and it is checked constructively: the oracle, re-run with some
u' in [u - 1e-6, u + 1e-6], must return the GPU's token. Kept sets must be equal, except at
a top-p boundary, where the exact (float64) cumulative mass at the cut is within BAND of
top_p, widened to the reference's own float32 normalizer error on that row. In that case
the reference's float32 sequential sum decides the cut. Probabilities
must agree within 1e-5 relative, or within 2e-6 relative of the float64 value when the
reference's sequential float32 normalizer is itself off by more than that.
"""
import numpy as np

import oracle as O

U_TOL = 1e-6
BAND = 1e-5
P_RTOL = 1e-5


def u_grid(u):
    return [float(np.float32(u + d)) for d in np.linspace(-U_TOL, U_TOL, 9)]


def exact_probs(s):
    s = s.astype(np.float64)
    m = np.max(s)
    if not np.isfinite(m):
        return None
    e = np.exp(s - m)
    return e / e.sum()


def top_p_band(s, top_p, lens, ref_sum=None):
    """True when the float64 cumulative mass near the cut is within the band of top_p: BAND,
    widened to what the reference's own float32 arithmetic demonstrably gets wrong on this
    row when its sequential normalizer `ref_sum` is given (twice the normalizer's relative
    error, which sequential summation of 10^4+ terms pushes past 1e-5 by dropping small
    terms, plus one rounding per cumsum step)."""
    pr = exact_probs(s)
    if pr is None:
        return False
    order = np.argsort(-pr, kind="stable")
    cum = np.cumsum(pr[order])
    lo, hi = max(min(lens) - 2, 0), min(max(lens), len(cum))
    band = BAND
    if ref_sum is not None:
        sv = s.astype(np.float64)
        fin = np.isfinite(sv)
        s_exact = float(np.sum(np.exp(sv[fin] - np.max(sv[fin]))))
        band = max(BAND, 2.0 * abs(float(ref_sum) / s_exact - 1.0) + hi * 6e-8)
    return bool(np.any(np.abs(cum[lo:hi] - top_p) <= band))


def band_draw(s, kept_len, u):
    """Tokens the reference draw returns at u' in [u - 1e-6, u + 1e-6] over the first
    kept_len elements of the float64 order (used when the kept length legitimately differs
    at a top-p boundary)."""
    pr = exact_probs(s)
    order = np.argsort(-pr, kind="stable")[:kept_len]
    cum = np.cumsum(pr[order])
    toks = set()
    for uu in u_grid(u):
        j = int(np.searchsorted(cum, uu * cum[-1], side="left"))
        toks.add(int(order[min(j, len(order) - 1)]))
    return toks if len(toks) == 1 else toks | {None}


def compare_target(cfg, gpu, orc, logits_f32=None, check_list=True):
    """gpu/orc: dicts of numpy arrays from target_rows. Returns (problems, stats)."""
    B = cfg["B"]
    prm = cfg["params"]
    problems, stats = [], dict(rows=B, u_exempt=0, band_exempt=0, listed_rows=0)
    for b in range(B):
        p = {k: float(prm[b][k]) if k != "top_k" else int(prm[b][k]) for k in prm.dtype.names if k != "reserved"}
        ok_, gk = int(orc["kind"][b]), int(gpu["kind"][b])
        if ok_ != gk:
            problems.append(f"row {b}: kind gpu={gk} oracle={ok_}")
            continue
        tok_g, tok_o = int(gpu["token"][b]), int(orc["token"][b])
        if ok_ == 0:
            if tok_g != tok_o:
                problems.append(f"row {b}: token target gpu={tok_g} oracle={tok_o}")
            continue
        # the softmax max is exact (x / T correctly rounded) and S within 2e-6 of an f64 sum
        if "stats" in gpu and "stats" in orc and p["temperature"] > 0.0:
            gm, om = np.float32(gpu["stats"][b, 0]), np.float32(orc["stats"][b, 0])
            if np.isfinite(om) and gm.view(np.uint32) != om.view(np.uint32):
                problems.append(f"row {b}: max gpu={gm!r} oracle={om!r}")
                continue
            if np.isfinite(om) and orc.get("s") is not None:
                sv = orc["s"][b].astype(np.float64)
                s_ex = float(np.sum(np.exp(sv[np.isfinite(sv)] - float(om))))
                if abs(float(gpu["stats"][b, 1]) - s_ex) > 2e-6 * s_ex:
                    problems.append(f"row {b}: sum gpu={float(gpu['stats'][b, 1])!r} f64={s_ex!r}")
                    continue
        kl_o, kl_g = int(orc["kept_len"][b]), int(gpu["kept_len"][b])
        band = False
        if kl_o != kl_g:
            ref_sum = orc["stats"][b, 1] if "stats" in orc else None
            if p["top_p"] < 1.0 and orc.get("s") is not None and \
                    top_p_band(orc["s"][b], p["top_p"], (kl_o, kl_g), ref_sum):
                band = True
                stats["band_exempt"] += 1
            else:
                problems.append(f"row {b}: kept_len gpu={kl_g} oracle={kl_o} params={p}")
                continue
        listed = int(gpu["listed"][b])
        if check_list and listed > 0 and not band:
            stats["listed_rows"] += 1
            ref_ids = orc["ids"][b, :kl_o]
            ref_w = orc["probs"][b, :kl_o]
            nz = ref_w > 0
            ri, rw = ref_ids[nz], ref_w[nz]
            gi, gw = gpu["ids"][b, :listed].astype(np.uint32), gpu["probs"][b, :listed]
            n = min(len(ri), len(gi))
            if len(gi) != min(len(ri), gpu["ids"].shape[1]) or not np.array_equal(gi[:n], ri[:n]):
                first = int(np.argmax(gi[:n] != ri[:n])) if n and not np.array_equal(gi[:n], ri[:n]) else n
                problems.append(f"row {b}: kept list differs at {first} (gpu {len(gi)} vs oracle {len(ri)}) params={p}")
                continue
            rel = np.abs(gw[:n] - rw[:n]) / np.maximum(rw[:n], 1e-38)
            if np.any(rel > P_RTOL):
                ex = exact_probs(orc["s"][b]) if orc.get("s") is not None else None
                bad = np.nonzero(rel > P_RTOL)[0]
                if ex is None or np.any(np.abs(gw[bad] - ex[gi[bad]]) / ex[gi[bad]] > 2e-6):
                    problems.append(f"row {b}: prob rel err {rel.max():.3g} at {int(bad[0])}")
                    continue
        if tok_g != tok_o:
            x = logits_f32[b] if logits_f32 is not None else None
            hist = cfg["hist"][cfg["hist_off"][b]:cfg["hist_off"][b + 1]]
            mask = None if cfg["mask"] is None else cfg["mask"][b]
            if x is not None and any(O.sample(x, hist, p, mask, uu) == tok_g for uu in u_grid(cfg["u"][b])):
                stats["u_exempt"] += 1
            elif band and band_draw(orc["s"][b], kl_g, cfg["u"][b]) == {tok_g}:
                stats["u_exempt"] += 1
            else:
                problems.append(f"row {b}: token gpu={tok_g} oracle={tok_o} u={cfg['u'][b]} params={p}")
    return problems, stats


def compare_exact(cfg, gpu, orc):
    """The exact bar: per row the GPU's target equals the oracle's bit for bit — kind, drawn
    token, kept length, the listed (id, probability) pairs (the kept entries with p > 0, up to
    the cap), the row maximum and the float32 normalizer. No exemption of any kind.
    Returns (problems, stats)."""
    B = cfg["B"]
    cap = gpu["ids"].shape[1]
    problems, stats = [], dict(rows=B, weights_rows=0, listed=0)
    for b in range(B):
        ok_, gk = int(orc["kind"][b]), int(gpu["kind"][b])
        if ok_ != gk:
            problems.append(f"row {b}: kind gpu={gk} oracle={ok_}")
            continue
        tg, to = int(gpu["token"][b]), int(orc["token"][b])
        if tg != to:
            problems.append(f"row {b}: token gpu={tg} oracle={to} u={float(cfg['u'][b])!r}")
        if ok_ == 0:
            continue
        stats["weights_rows"] += 1
        om, gm = np.float32(orc["stats"][b, 0]), np.float32(gpu["stats"][b, 0])
        os_, gs = np.float32(orc["stats"][b, 1]), np.float32(gpu["stats"][b, 1])
        if np.isfinite(om) and om.view(np.uint32) != gm.view(np.uint32):
            problems.append(f"row {b}: max gpu={gm!r} oracle={om!r}")
        if np.isfinite(os_) and os_.view(np.uint32) != gs.view(np.uint32):
            problems.append(f"row {b}: normalizer gpu={gs!r} oracle={os_!r}")
        kl_o, kl_g = int(orc["kept_len"][b]), int(gpu["kept_len"][b])
        if kl_o != kl_g:
            problems.append(f"row {b}: kept_len gpu={kl_g} oracle={kl_o}")
            continue
        n = min(kl_o, orc["ids"].shape[1])
        rw = orc["probs"][b, :n]
        ri = orc["ids"][b, :n][rw > 0][:cap]
        rw = rw[rw > 0][:cap]
        listed = int(gpu["listed"][b])
        if listed != len(ri):
            problems.append(f"row {b}: listed gpu={listed} oracle={len(ri)} (kept {kl_o})")
            continue
        gi = gpu["ids"][b, :listed].astype(np.uint32)
        gw = gpu["probs"][b, :listed].astype(np.float32)
        if not np.array_equal(gi, ri.astype(np.uint32)):
            first = int(np.argmax(gi != ri))
            problems.append(f"row {b}: kept ids differ at {first}: gpu {int(gi[first])} oracle {int(ri[first])}")
            continue
        if not np.array_equal(gw.view(np.uint32), rw.astype(np.float32).view(np.uint32)):
            first = int(np.argmax(gw.view(np.uint32) != rw.astype(np.float32).view(np.uint32)))
            problems.append(f"row {b}: probability {first} gpu={gw[first]!r} oracle={rw[first]!r}")
            continue
        stats["listed"] += listed
    return problems, stats
