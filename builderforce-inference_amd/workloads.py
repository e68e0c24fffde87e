"""Seeded synthetic inputs for the five benchmark configurations of the sampling path.

Each generator returns numpy arrays (host); `to_device` moves them into HBM as the tensors
bfi_smp.Sampler takes. `scale_v` shrinks the vocabulary for parity tests the CPU oracle
finishes in seconds; everything else keeps the configuration's shape and distributions.

  C1  B=1,   V=151936 f32 ~N(0,2.5), 8 ids +10, rep 1.1 over 64 uniform ids,
      T 0.7 / k 40 / p 0.95 (and a greedy variant)
  C2  B=64,  V=151936 f32 ~N(0,2.5) + 1..16 peaked ids (+6..+12); per-row T U[0.2,1.5],
      k in {0,20,50,100}, p U[0.8,1.0], min-p 0.05; 512-id Zipf(1.1) histories with
      repetition 1.1, presence 0.5, frequency 0.3
  C2M C2 under C3's grammar allow-masks (the full-feature row: penalties, top-k/top-p/min-p
      and a mask)
  C3  B=32,  V=151936 f32 as C2 logits, packed allow-mask with allowed fraction
      log-uniform in [0.1%, 30%] in runs of 1..64 ids (some rows allow exactly 1 id);
      T 1.0 / p 0.9
  C4  16 sequences x (4 drafts + 1) = 80 rows, V=151936 f32; drafts random ids, half forced
      to the row argmax; T 0.8 / p 0.95 (and greedy)
  C5  B=256, V=262144 bf16 ~N(0,3) with 5% of ids +4; top-p 0.9, no top-k, min-p 0, T 1.0;
      repetition 1.05 over 1024-id Zipf(1.1) histories
"""
from __future__ import annotations

import numpy as np

from bfi_smp import PARAMS_DTYPE, params_array

QWEN3_V = 151936


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 (as uint16 bits); inputs are finite."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def zipf_table(V: int, s: float, rng) -> tuple[np.ndarray, np.ndarray]:
    """Inverse-CDF table of Zipf(s) over ranks 1..V and a fixed rank -> id permutation."""
    w = np.arange(1, V + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    perm = rng.permutation(V).astype(np.uint32)
    return cdf, perm


def zipf_histories(rng, B: int, H: int, V: int, s: float = 1.1):
    cdf, perm = zipf_table(V, s, rng)
    u = rng.random((B, H))
    ranks = np.searchsorted(cdf, u, side="right").clip(0, V - 1)
    hist = perm[ranks].astype(np.uint32).reshape(-1)
    off = np.arange(B + 1, dtype=np.int64) * H
    return hist, off


def peaked_logits(rng, B, V, sigma=2.5, n_peak=(1, 16), boost=(6.0, 12.0)):
    x = (rng.standard_normal((B, V)) * sigma).astype(np.float32)
    for b in range(B):
        n = int(rng.integers(n_peak[0], n_peak[1] + 1))
        ids = rng.choice(V, n, replace=False)
        x[b, ids] += rng.uniform(boost[0], boost[1], n).astype(np.float32)
    return x


def run_masks(rng, B, V, frac=(0.001, 0.30), runs=(1, 64), single_rows=(0,)):
    W = (V + 31) // 32
    m = np.zeros((B, W), np.uint32)
    for b in range(B):
        allowed = np.zeros(V, bool)
        if b in single_rows:
            allowed[rng.integers(0, V)] = True
        else:
            target = int(np.exp(rng.uniform(np.log(frac[0]), np.log(frac[1]))) * V)
            target = max(target, 1)
            while allowed.sum() < target:
                start = int(rng.integers(0, V))
                ln = int(rng.integers(runs[0], runs[1] + 1))
                allowed[start : start + ln] = True
        idx = np.nonzero(allowed)[0]
        np.bitwise_or.at(m[b], idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return m


def config(name: str, seed: int = 0, scale_v: float = 1.0, greedy: bool = False) -> dict:
    rng = np.random.default_rng([seed, {"C1": 1, "C2": 2, "C3": 3, "C4": 4, "C5": 5, "C2M": 6}[name]])
    out = dict(name=name, mask=None, dtype="f32")
    if name == "C1":
        V = max(int(QWEN3_V * scale_v), 64)
        B = 1
        x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
        x[0, rng.choice(V, 8, replace=False)] += 10.0
        hist = rng.integers(0, V, 64).astype(np.uint32)
        off = np.array([0, 64], np.int64)
        p = dict(temperature=0.0 if greedy else 0.7, top_k=40, top_p=0.95, repeat_penalty=1.1)
        params = params_array([p])
    elif name in ("C2", "C2M"):
        V = max(int(QWEN3_V * scale_v), 256)
        B = 64
        x = peaked_logits(rng, B, V)
        hist, off = zipf_histories(rng, B, 512, V)
        rows = []
        for b in range(B):
            rows.append(dict(
                temperature=0.0 if greedy else float(rng.uniform(0.2, 1.5)),
                top_k=int(rng.choice([0, 20, 50, 100])),
                top_p=float(rng.uniform(0.8, 1.0)),
                min_p=0.05,
                repeat_penalty=1.1,
                presence_penalty=0.5,
                frequency_penalty=0.3,
            ))
        params = params_array(rows)
        if name == "C2M":  # the same rows under a grammar allow-mask (C3's masks)
            out["mask"] = run_masks(rng, B, V, single_rows=(0, 7))
    elif name == "C3":
        V = max(int(QWEN3_V * scale_v), 256)
        B = 32
        x = peaked_logits(rng, B, V)
        hist = np.zeros(0, np.uint32)
        off = np.zeros(B + 1, np.int64)
        out["mask"] = run_masks(rng, B, V, single_rows=(0, 7))
        params = params_array([dict(temperature=0.0 if greedy else 1.0, top_p=0.9)] * B)
    elif name == "C4":
        V = max(int(QWEN3_V * scale_v), 256)
        S, K = 16, 4
        B = S * (K + 1)
        x = peaked_logits(rng, B, V)
        drafts = rng.integers(0, V, (S, K)).astype(np.uint32)
        for s in range(S):
            for i in range(K):
                if rng.random() < 0.5:
                    drafts[s, i] = np.argmax(x[s * (K + 1) + i])
        hist, off = zipf_histories(rng, S, 64, V)
        params = params_array([dict(temperature=0.0 if greedy else 0.8, top_p=0.95)] * S)
        out.update(n_seq=S, rows_per_seq=K + 1, drafts=drafts, draft_len=np.full(S, K, np.int32),
                   u_pairs=rng.random((S, K, 2)).astype(np.float32), u_bonus=rng.random(S).astype(np.float32))
    elif name == "C5":
        V = max(int(262144 * scale_v), 256)
        B = 256
        xf = (rng.standard_normal((B, V)) * 3.0).astype(np.float32)
        heavy = rng.random((B, V)) < 0.05
        xf[heavy] += 4.0
        x = f32_to_bf16_bits(xf).reshape(B, V)
        out["dtype"] = "bf16"
        hist, off = zipf_histories(rng, B, 1024, V)
        params = params_array([dict(temperature=0.0 if greedy else 1.0, top_p=0.9, repeat_penalty=1.05)] * B)
    else:
        raise ValueError(name)
    out.update(V=V, B=B, logits=x, hist=hist, hist_off=off, params=params,
               u=rng.random(B).astype(np.float32))
    return out


def algorithmic_bytes(cfg: dict) -> int:
    """Bytes one call must move at minimum: logits + mask + history + params + u + token."""
    B, V = cfg["B"], cfg["V"]
    esz = 2 if cfg["dtype"] == "bf16" else 4
    n = B * V * esz
    if cfg["mask"] is not None:
        n += cfg["mask"].nbytes
    n += int(cfg["hist"].nbytes) + int(cfg["hist_off"].nbytes)
    n += cfg["params"].nbytes + B * 4 + B * 4
    return n


def to_device(cfg: dict, device="cuda:0") -> dict:
    import torch

    d = {}
    if cfg["dtype"] == "bf16":
        d["logits"] = torch.from_numpy(cfg["logits"].view(np.int16)).to(device).view(torch.bfloat16)
    else:
        d["logits"] = torch.from_numpy(cfg["logits"]).to(device)
    d["params"] = torch.from_numpy(np.ascontiguousarray(cfg["params"]).view(np.uint8).copy()).to(device)
    d["hist"] = torch.from_numpy(cfg["hist"].view(np.int32).copy()).to(device) if cfg["hist"].size else \
        torch.zeros(1, dtype=torch.int32, device=device)
    d["hist_off"] = torch.from_numpy(cfg["hist_off"]).to(device)
    d["u"] = torch.from_numpy(cfg["u"]).to(device)
    d["mask"] = None if cfg["mask"] is None else torch.from_numpy(cfg["mask"].view(np.int32).copy()).to(device)
    d["out"] = torch.zeros(cfg["B"], dtype=torch.int32, device=device)
    if "drafts" in cfg:
        d["drafts"] = torch.from_numpy(cfg["drafts"].view(np.int32).copy()).to(device)
        d["draft_len"] = torch.from_numpy(cfg["draft_len"]).to(device)
        d["u_pairs"] = torch.from_numpy(cfg["u_pairs"].reshape(-1)).to(device)
        d["u_bonus"] = torch.from_numpy(cfg["u_bonus"]).to(device)
        d["out_accepted"] = torch.zeros(cfg["n_seq"], dtype=torch.int32, device=device)
        d["out_next"] = torch.zeros(cfg["n_seq"], dtype=torch.int32, device=device)
    return d


# ---- the allow-mask producer's workload (include/bfi_mask.h) ------------------------------

MASK_SO_FAR = b'{"name": "lookup", "arguments": {"query": "weather in '
MASK_TOOLS = dict(tool_choice=3, tool_name=b"lookup", tool_names=[b"lookup", b"search", b"list_files"])


def synthetic_vocab(V: int = 151936, seed: int = 0) -> list:
    """V decoded pieces shaped like a BPE vocabulary: 1-16 bytes (mean about 6), mostly
    letters with a leading space, plus digits, JSON punctuation and some UTF-8 (no tokenizer
    files are available, so the texts are synthetic)."""
    rng = np.random.default_rng(seed)
    letters = np.frombuffer(b"abcdefghijklmnopqrstuvwxyz", np.uint8)
    punct = [b"{", b"}", b"[", b"]", b'"', b":", b",", b"\\", b'":', b'{"', b'"}', b"\n", b"  ", b"\t"]
    lens = np.clip(rng.geometric(0.18, V), 1, 16)
    out = []
    for i in range(V):
        r = rng.random()
        if r < 0.08:
            out.append(punct[rng.integers(len(punct))] + (b'"' if rng.random() < 0.2 else b""))
        elif r < 0.12:
            out.append(str(int(rng.integers(0, 1000))).encode())
        elif r < 0.15:
            out.append("é✓日本ü"[rng.integers(5)].encode() * int(rng.integers(1, 3)))
        else:
            w = bytes(letters[rng.integers(0, 26, int(lens[i]))])
            out.append((b" " + w) if rng.random() < 0.5 else w)
    return out
