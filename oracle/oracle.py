"""TEST INFRASTRUCTURE ONLY — ctypes binding of the C oracle (libbfi_oracle.so).

The oracle restates crates/bfi-runtime/src/sample.rs and engine/spec.rs of the reference
(see bfi_oracle.h for what pins each function). Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module; the product path never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbfi_oracle.so")

PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_k", "<i4"),
        ("top_p", "<f4"),
        ("min_p", "<f4"),
        ("repeat_penalty", "<f4"),
        ("presence_penalty", "<f4"),
        ("frequency_penalty", "<f4"),
        ("reserved", "<u4"),
    ]
)

# SampleParams::default() numeric fields (sample.rs:33-50)
DEFAULTS = dict(
    temperature=0.0,
    top_k=0,
    top_p=1.0,
    min_p=0.0,
    repeat_penalty=1.0,
    presence_penalty=0.0,
    frequency_penalty=0.0,
)


class _Info(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("token", ctypes.c_uint32),
        ("len", ctypes.c_int64),
        ("max", ctypes.c_float),
        ("sum", ctypes.c_float),
        ("len_k", ctypes.c_int64),
        ("len_p", ctypes.c_int64),
        ("len_m", ctypes.c_int64),
        ("sorted", ctypes.c_int32),
        ("minp_fallback", ctypes.c_int32),
    ]


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


def use_library(path):
    """Switches this module to another build of the oracle (the mutation tests load
    variants with a planted mistake); returns the previous handle for restore_library."""
    global _lib
    prev = _lib
    _lib = None
    lib(path)
    return prev


def restore_library(handle):
    global _lib
    _lib = handle


def lib(path=None):
    global _lib
    if _lib is None:
        path = path or LIB_PATH
        if path == LIB_PATH and not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        L.orc_rng_next.restype = ctypes.c_uint64
        L.orc_rng_next.argtypes = [P]
        L.orc_rng_f32.restype = ctypes.c_float
        L.orc_rng_f32.argtypes = [P]
        L.orc_slot_rng_seed.restype = ctypes.c_uint64
        L.orc_slot_rng_seed.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.orc_argmax.restype = ctypes.c_uint32
        L.orc_argmax.argtypes = [P, P, ctypes.c_size_t]
        L.orc_draw.restype = ctypes.c_uint32
        L.orc_draw.argtypes = [P, P, ctypes.c_size_t, ctypes.c_float]
        L.orc_target.restype = ctypes.c_int
        L.orc_target.argtypes = [P, ctypes.c_size_t, P, ctypes.c_size_t, P, P, P, P, P, P]
        L.orc_sample.restype = ctypes.c_uint32
        L.orc_sample.argtypes = [P, ctypes.c_size_t, P, ctypes.c_size_t, P, P, ctypes.c_float]
        L.orc_judge.restype = ctypes.c_int
        L.orc_judge.argtypes = [
            ctypes.c_int32,
            ctypes.c_uint32,
            P,
            P,
            ctypes.c_size_t,
            ctypes.c_uint32,
            ctypes.c_float,
            ctypes.c_float,
            P,
        ]
        L.orc_draft.restype = ctypes.c_size_t
        L.orc_draft.argtypes = [P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, P]
        L.orc_parse_id_union.restype = ctypes.c_int
        L.orc_parse_id_union.argtypes = [ctypes.c_char_p, ctypes.c_int64, P]
        I64 = ctypes.c_int64
        L.orc_sample_rows.restype = None
        L.orc_sample_rows.argtypes = [I64, I64, P, ctypes.c_int, I64, P, P, P, P, I64, P, P, ctypes.c_int]
        L.orc_target_rows.restype = None
        L.orc_target_rows.argtypes = [
            I64, I64, P, ctypes.c_int, I64, P, P, P, P, I64, P, P, P, P, P, P, I64, P, P, ctypes.c_int
        ]
        L.orc_verify_seq.restype = None
        L.orc_rms_norm.argtypes = [P, P, ctypes.c_int, ctypes.c_float, I64, I64, P]
        L.orc_rms_norm.restype = None
        L.orc_matmul_f32.argtypes = [P, P, I64, I64, I64, P]
        L.orc_matmul_f32.restype = None
        L.orc_dequant.argtypes = [ctypes.c_int, P, I64, P]
        L.orc_dequant.restype = ctypes.c_int
        L.orc_matmul_blocked.argtypes = [P, P, I64, I64, I64, I64, P]
        L.orc_matmul_blocked.restype = None
        L.orc_matmul_signs.argtypes = [P, P, I64, I64, I64, I64, P]
        L.orc_matmul_signs.restype = None
        L.orc_verify_seq.argtypes = [
            P, ctypes.c_int, I64, I64, P, P, ctypes.c_size_t, P, ctypes.c_size_t, P, I64, P,
            ctypes.c_float, P, P,
        ]
        _lib = L
    return _lib


def rms_norm(x, w, eps: float, w_per_row: bool = False):
    """cpu.rs:92-120 over rows of x (float32 [n, d])."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    n, d = x.shape
    out = np.empty_like(x)
    lib().orc_rms_norm(_ptr(x), _ptr(w), 1 if w_per_row else 0, ctypes.c_float(eps), n, d, _ptr(out))
    return out


def matmul_f32(w, x):
    """cpu.rs:498-514: [n_tokens, n_out] = x @ w.T with sequential f32 dots."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    lib().orc_matmul_f32(_ptr(w), _ptr(x), x.shape[0], w.shape[0], w.shape[1], _ptr(out))
    return out


def dequant(ggml_type: int, src, n: int):
    """A GGML tensor's first n weights (src: its bytes) to float32 (types/<format>.rs)."""
    src = np.ascontiguousarray(src, np.uint8)
    out = np.empty(n, np.float32)
    if lib().orc_dequant(int(ggml_type), _ptr(src), n, _ptr(out)) != 0:
        raise ValueError(f"GGML type {ggml_type} is not restated")
    return out


def matmul_blocked(w, x, block: int):
    """matmul_quant's dot order (cpu.rs:550-563) over dequantized weights: blocks of `block`
    products summed from -0.0, the blocks from +0.0 (block 0: one dot over the row)."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    lib().orc_matmul_blocked(_ptr(w), _ptr(x), x.shape[0], w.shape[0], w.shape[1], int(block), _ptr(out))
    return out


def matmul_signs(w, x, block: int = 128):
    """The Q1_0 row dot (simd.rs:74-80, q1_0.rs:48-64) over dequantized weights (+-d): each
    block's activations summed with their weight's sign, times the block's scale."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    lib().orc_matmul_signs(_ptr(w), _ptr(x), x.shape[0], w.shape[0], w.shape[1], int(block), _ptr(out))
    return out


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def params_array(rows) -> np.ndarray:
    """Structured array of bfi_smp_row_params from a dict or a list of dicts."""
    if isinstance(rows, dict):
        rows = [rows]
    out = np.zeros(len(rows), dtype=PARAMS_DTYPE)
    for i, r in enumerate(rows):
        d = dict(DEFAULTS)
        d.update(r)
        for k, v in d.items():
            out[i][k] = v
    return out


def rng_next(state: int):
    s = ctypes.c_uint64(state)
    v = lib().orc_rng_next(ctypes.byref(s))
    return v, s.value


def rng_f32(state: int):
    s = ctypes.c_uint64(state)
    v = lib().orc_rng_f32(ctypes.byref(s))
    return v, s.value


def slot_rng_seed(seed: int, prompt_len: int) -> int:
    return lib().orc_slot_rng_seed(seed, prompt_len)


def argmax(v) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return lib().orc_argmax(None, _ptr(v), v.size)


def draw(ids, w, u: float) -> int:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    return lib().orc_draw(_ptr(ids), _ptr(w), w.size, u)


def _mask_arg(mask):
    return None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)


def target(logits, prev, params: dict, mask=None, want_s=False):
    """Returns dict(kind, token, ids, w, info..., s)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    V = x.size
    h = np.ascontiguousarray(prev, dtype=np.uint32)
    p = params_array(params)
    m = _mask_arg(mask)
    ids = np.zeros(max(V, 1), dtype=np.uint32)
    w = np.zeros(max(V, 1), dtype=np.float32)
    s = np.zeros(max(V, 1), dtype=np.float32) if want_s else None
    info = _Info()
    rc = lib().orc_target(
        _ptr(x), V, _ptr(h), h.size, _ptr(p), _ptr(m), _ptr(ids), _ptr(w), _ptr(s), ctypes.byref(info)
    )
    assert rc == 0
    out = dict(
        kind=info.kind,
        token=info.token,
        len=info.len,
        max=info.max,
        sum=info.sum,
        len_k=info.len_k,
        len_p=info.len_p,
        len_m=info.len_m,
        sorted=info.sorted,
        minp_fallback=info.minp_fallback,
    )
    if info.kind == 1:
        out["ids"] = ids[: info.len].copy()
        out["w"] = w[: info.len].copy()
    else:
        out["ids"] = np.zeros(0, np.uint32)
        out["w"] = np.zeros(0, np.float32)
    if want_s:
        out["s"] = s[:V].copy()
    return out


def sample(logits, prev, params: dict, mask=None, u: float = 0.0) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(prev, dtype=np.uint32)
    p = params_array(params)
    return lib().orc_sample(_ptr(x), x.size, _ptr(h), h.size, _ptr(p), _ptr(_mask_arg(mask)), u)


def sample_seeded(logits, prev, params: dict, seed: int, mask=None) -> int:
    """sample() exactly as the reference calls it: u = Rng(seed).f32() (sample.rs:307)."""
    u, _ = rng_f32(seed)
    return sample(logits, prev, params, mask, u)


def judge(tgt, d: int, u: float, u2: float):
    """tgt: ('token', t) or ('weights', [(id, w), ...]) -> ('accept', None) / ('reject', t)."""
    rej = ctypes.c_uint32(0)
    if tgt[0] == "token":
        acc = lib().orc_judge(0, tgt[1], None, None, 0, d, u, u2, ctypes.byref(rej))
    else:
        ids = np.array([a for a, _ in tgt[1]], dtype=np.uint32)
        w = np.array([b for _, b in tgt[1]], dtype=np.float32)
        acc = lib().orc_judge(1, 0, _ptr(ids), _ptr(w), ids.size, d, u, u2, ctypes.byref(rej))
    return ("accept", None) if acc else ("reject", rej.value)


def draft(ctx, k: int, ngram_max: int = 3, ngram_min: int = 2):
    c = np.ascontiguousarray(ctx, dtype=np.uint32)
    out = np.zeros(max(k, 1), dtype=np.uint32)
    n = lib().orc_draft(_ptr(c), c.size, k, ngram_max, ngram_min, _ptr(out))
    return [int(v) for v in out[:n]]


def parse_id_union(grammar: str, n_vocab: int):
    m = np.zeros((n_vocab + 31) // 32, dtype=np.uint32)
    ok = lib().orc_parse_id_union(grammar.encode(), n_vocab, _ptr(m))
    return m if ok else None


def sample_rows(logits, params, hist, hist_off, u, mask=None, dtype=0, threads=1):
    """logits: [B, V] f32 array (or uint16 bf16 bits when dtype=1)."""
    x = np.ascontiguousarray(logits)
    B, V = x.shape
    p = np.ascontiguousarray(params)
    h = np.ascontiguousarray(hist, dtype=np.uint32)
    ho = np.ascontiguousarray(hist_off, dtype=np.int64)
    uu = np.ascontiguousarray(u, dtype=np.float32)
    m = _mask_arg(mask)
    ms = 0 if m is None else m.shape[1]
    out = np.zeros(B, dtype=np.uint32)
    lib().orc_sample_rows(B, V, _ptr(x), dtype, V, _ptr(p), _ptr(h), _ptr(ho), _ptr(m), ms, _ptr(uu), _ptr(out), threads)
    return out


def target_rows(logits, params, hist, hist_off, u, mask=None, dtype=0, cap=None, threads=8, want_s=False):
    x = np.ascontiguousarray(logits)
    B, V = x.shape
    cap = V if cap is None else cap
    p = np.ascontiguousarray(params)
    h = np.ascontiguousarray(hist, dtype=np.uint32)
    ho = np.ascontiguousarray(hist_off, dtype=np.int64)
    uu = np.ascontiguousarray(u, dtype=np.float32)
    m = _mask_arg(mask)
    ms = 0 if m is None else m.shape[1]
    tok = np.zeros(B, np.uint32)
    kind = np.zeros(B, np.int32)
    kl = np.zeros(B, np.int32)
    ids = np.zeros((B, cap), np.uint32)
    probs = np.zeros((B, cap), np.float32)
    s = np.zeros((B, V), np.float32) if want_s else None
    stats = np.zeros((B, 8), np.float32)
    lib().orc_target_rows(
        B, V, _ptr(x), dtype, V, _ptr(p), _ptr(h), _ptr(ho), _ptr(m), ms, _ptr(uu),
        _ptr(tok), _ptr(kind), _ptr(kl), _ptr(ids), _ptr(probs), cap, _ptr(s), _ptr(stats), threads,
    )
    return dict(token=tok, kind=kind, kept_len=kl, ids=ids, probs=probs, s=s, stats=stats)


def verify_seq(rows, params: dict, hist, drafts, u_pairs, u_bonus: float, masks=None, dtype=0):
    """rows: [draft_len+1, V]; returns (accepted, next)."""
    x = np.ascontiguousarray(rows)
    V = x.shape[1]
    p = params_array(params)
    h = np.ascontiguousarray(hist, dtype=np.uint32)
    d = np.ascontiguousarray(drafts, dtype=np.uint32)
    up = np.ascontiguousarray(u_pairs, dtype=np.float32)
    m = _mask_arg(masks)
    ms = 0 if m is None else m.shape[1]
    acc = ctypes.c_int32(0)
    nxt = ctypes.c_uint32(0)
    lib().orc_verify_seq(
        _ptr(x), dtype, V, V, _ptr(p), _ptr(h), h.size, _ptr(d), d.size, _ptr(m), ms, _ptr(up),
        u_bonus, ctypes.byref(acc), ctypes.byref(nxt),
    )
    return acc.value, nxt.value
