"""Comparison of GPU results with the CPU oracle: the exact bar of the sampling path.

The GPU reproduces the reference's float32 arithmetic (its sequential normalizer, top-p
cumulative sums and draw sums, sample.rs:312-424, spec.rs:79-97), so its results are the
oracle's bit for bit: kind, drawn token, kept length, the listed (id, probability) pairs,
the row maximum and the float32 normalizer. No tolerance and no exemption of any kind.
"""
import numpy as np


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
