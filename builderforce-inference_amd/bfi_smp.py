"""ctypes binding of libbfi_sampler.so (include/bfi_sampler.h).

PyTorch supplies device memory and the stream; every call goes through the C ABI to the
HIP kernels. There is no CPU fallback: a missing library or device raises.
Names follow the reference (crates/bfi-runtime/src/sample.rs `sample`, `target`;
engine/spec.rs `judge` via `verify`).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbfi_sampler.so")

F32, BF16 = 0, 1
TARGET_TOKEN, TARGET_WEIGHTS = 0, 1

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
# SampleParams::default() (sample.rs:33-50), numeric fields
DEFAULTS = dict(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0,
                presence_penalty=0.0, frequency_penalty=0.0)

_lib = None


class SamplerError(RuntimeError):
    pass


def lib():
    """Loads the HIP library; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SamplerError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C {HERE})")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.bfi_smp_create.argtypes = [I32, ctypes.POINTER(P)]
        L.bfi_smp_destroy.argtypes = [P]
        L.bfi_smp_destroy.restype = None
        L.bfi_smp_last_error.argtypes = [P]
        L.bfi_smp_last_error.restype = ctypes.c_char_p
        L.bfi_smp_abi_version.restype = I32
        L.bfi_smp_set_tracing.argtypes = [P, I32]
        L.bfi_smp_trace.argtypes = [P, P, I64]
        L.bfi_smp_trace.restype = I64
        L.bfi_smp_set_profiling.argtypes = [P, I32]
        L.bfi_smp_profile.argtypes = [P, P, P]
        L.bfi_smp_sample_rows.argtypes = [P, P, I32, I64, I64, I64, P, P, P, P, I64, P, P, P]
        L.bfi_smp_sample_rows_noalloc.argtypes = [P, P, I32, I64, I64, I64, P, P, P, P, I64, P, P, P]
        L.bfi_smp_target_rows.argtypes = [P, P, I32, I64, I64, I64, P, P, P, P, I64, P, P, P, P, P, P, P, I64, P, P]
        L.bfi_smp_verify.argtypes = [P, P, I32, I64, I64, I64, I64, P, P, P, P, P, P, I64, P, P, P, P, P]
        L.bfi_smp_sample_host.argtypes = [P, P, I64, P, I64, P, P, ctypes.c_float, P]
        L.bfi_smp_head.argtypes = [P, P, P, I32, ctypes.c_float, P, I64, I64, I64, P, P]
        L.bfi_smp_dequant.argtypes = [P, I32, P, I64, P, P]
        L.bfi_smp_head_typed.argtypes = [P, P, P, I32, ctypes.c_float, P, I32, I64, I64, I64, P, P]
        L.bfi_smp_head_typed_sample_rows.argtypes = [P, P, P, I32, ctypes.c_float, P, I32, I64, I64, I64, P, P, P,
                                                     P, I64, P, P, P]
        L.bfi_smp_head_sample_rows.argtypes = [P, P, P, I32, ctypes.c_float, P, I64, I64, I64, P, P, P, P, I64, P, P,
                                               P]
        L.bfi_rng_next_u64.argtypes = [P]
        L.bfi_rng_next_u64.restype = ctypes.c_uint64
        L.bfi_rng_f32.argtypes = [P]
        L.bfi_rng_f32.restype = ctypes.c_float
        L.bfi_slot_rng_seed.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.bfi_slot_rng_seed.restype = ctypes.c_uint64
        L.bfi_draft.argtypes = [P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, P]
        L.bfi_draft.restype = ctypes.c_size_t
        L.bfi_parse_id_union.argtypes = [ctypes.c_char_p, I64, P]
        L.bfi_parse_id_union.restype = I32
        L.bfi_spec_replay.argtypes = [P, P, ctypes.c_size_t, ctypes.c_int32, ctypes.c_uint32, I64, ctypes.c_size_t,
                                      ctypes.c_size_t, P, P, P, P, P, P]
        # allow-mask producer (include/bfi_mask.h)
        L.bfi_mask_create.argtypes = [I32, ctypes.POINTER(P)]
        L.bfi_mask_destroy.argtypes = [P]
        L.bfi_mask_destroy.restype = None
        L.bfi_mask_error.argtypes = [P]
        L.bfi_mask_error.restype = ctypes.c_char_p
        L.bfi_mask_set_vocab.argtypes = [P, P, P, I64]
        L.bfi_mask_build.argtypes = [P, P, I64, ctypes.POINTER(Constraint), P, ctypes.POINTER(ctypes.c_int32), P]
        # prefix cache (include/bfi_prefix.h)
        U64 = ctypes.c_uint64
        L.bfi_pc_create.argtypes = [I32, U64, ctypes.POINTER(P)]
        L.bfi_pc_destroy.argtypes = [P]
        L.bfi_pc_destroy.restype = None
        L.bfi_pc_last_error.argtypes = [P]
        L.bfi_pc_last_error.restype = ctypes.c_char_p
        L.bfi_pc_lookup.argtypes = [P, P, U64, ctypes.POINTER(PCHit), ctypes.POINTER(I32)]
        L.bfi_pc_restore.argtypes = [P, ctypes.POINTER(PCHit), ctypes.POINTER(PCState), ctypes.POINTER(U64),
                                     ctypes.POINTER(I32), ctypes.POINTER(I32), P]
        L.bfi_pc_insert.argtypes = [P, P, U64, ctypes.POINTER(PCState), P]
        for f in ("bfi_pc_used_bytes", "bfi_pc_len", "bfi_pc_forwarded"):
            getattr(L, f).argtypes = [P]
            getattr(L, f).restype = U64
        L.bfi_pc_note_forward.argtypes = [P, U64]
        L.bfi_pc_note_forward.restype = None
        L.bfi_pc_clear.argtypes = [P]
        L.bfi_pc_clear.restype = None
        _lib = L
    return _lib


TOOL_NONE, TOOL_AUTO, TOOL_REQUIRED, TOOL_NAMED = 0, 1, 2, 3


class Constraint(ctypes.Structure):
    """bfi_constraint (include/bfi_mask.h): the constraint fields of SampleParams."""
    _fields_ = [
        ("json_object", ctypes.c_int32),
        ("tool_choice", ctypes.c_int32),
        ("tool_name", ctypes.c_void_p),
        ("tool_name_len", ctypes.c_int64),
        ("tool_names", ctypes.c_void_p),
        ("tool_name_lens", ctypes.c_void_p),
        ("n_tool_names", ctypes.c_int32),
        ("grammar", ctypes.c_void_p),
        ("grammar_len", ctypes.c_int64),
    ]


class PCTensor(ctypes.Structure):
    """bfi_pc_tensor (include/bfi_prefix.h)."""
    _fields_ = [("data", ctypes.c_void_p), ("row_bytes", ctypes.c_uint64), ("rows", ctypes.c_uint64)]


class PCState(ctypes.Structure):
    """bfi_pc_state (include/bfi_prefix.h)."""
    _fields_ = [("n", ctypes.c_uint64), ("kv", ctypes.c_void_p), ("n_kv", ctypes.c_uint64),
                ("rec", ctypes.c_void_p), ("n_rec", ctypes.c_uint64), ("logits", ctypes.c_void_p),
                ("n_logits", ctypes.c_uint64)]


class PCHit(ctypes.Structure):
    """bfi_pc_hit (include/bfi_prefix.h)."""
    _fields_ = [("id", ctypes.c_uint64), ("matched", ctypes.c_uint64), ("restore", ctypes.c_uint64)]


def params_array(rows) -> np.ndarray:
    if isinstance(rows, dict):
        rows = [rows]
    out = np.zeros(len(rows), dtype=PARAMS_DTYPE)
    for i, r in enumerate(rows):
        d = dict(DEFAULTS)
        d.update(r)
        for k, v in d.items():
            out[i][k] = v
    return out


def _np_ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---- host helpers (no GPU) ---------------------------------------------------------------


def rng_f32(state: int):
    s = ctypes.c_uint64(state)
    v = lib().bfi_rng_f32(ctypes.byref(s))
    return v, s.value


def rng_next_u64(state: int):
    s = ctypes.c_uint64(state)
    v = lib().bfi_rng_next_u64(ctypes.byref(s))
    return v, s.value


def slot_rng_seed(seed: int, prompt_len: int) -> int:
    return lib().bfi_slot_rng_seed(seed, prompt_len)


def draft(ctx, k, ngram_max=3, ngram_min=2):
    c = np.ascontiguousarray(ctx, dtype=np.uint32)
    out = np.zeros(max(k, 1), np.uint32)
    n = lib().bfi_draft(_np_ptr(c), c.size, k, ngram_max, ngram_min, _np_ptr(out))
    return [int(x) for x in out[:n]]


def parse_id_union(grammar: str, n_vocab: int):
    m = np.zeros(max((n_vocab + 31) // 32, 1), np.uint32)
    ok = lib().bfi_parse_id_union(grammar.encode(), n_vocab, _np_ptr(m))
    return m[: (n_vocab + 31) // 32] if ok else None


def spec_replay(drafted, kernel_accepted, kernel_next, eos, generated, max_tokens, rng_state, closes_tool=None):
    """bfi_spec_replay; closes_tool: per draft, whether appending it completes a tool call."""
    d = np.ascontiguousarray(drafted, dtype=np.uint32)
    stops = None if closes_tool is None else np.ascontiguousarray(closes_tool, dtype=np.uint8)
    pushed = np.zeros(max(d.size, 1), np.uint32)
    st = ctypes.c_uint64(rng_state)
    n_pushed, acc = ctypes.c_size_t(0), ctypes.c_size_t(0)
    done, pend = ctypes.c_int(0), ctypes.c_int64(0)
    rc = lib().bfi_spec_replay(_np_ptr(d), None if stops is None else _np_ptr(stops), d.size, kernel_accepted,
                               kernel_next, -1 if eos is None else eos,
                               generated, max_tokens, ctypes.byref(st), _np_ptr(pushed), ctypes.byref(n_pushed),
                               ctypes.byref(acc), ctypes.byref(done), ctypes.byref(pend))
    if rc:
        raise SamplerError("bfi_spec_replay failed")
    return dict(pushed=[int(x) for x in pushed[: n_pushed.value]], accepted=acc.value, done=bool(done.value),
                pending=None if pend.value < 0 else pend.value, rng_state=st.value)


# ---- device sampler ----------------------------------------------------------------------


def _dptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Sampler:
    """One bfi_smp_ctx on a HIP device (not for concurrent use)."""

    def __init__(self, device: int = 0):
        self._L = lib()
        self._ctx = ctypes.c_void_p()
        rc = self._L.bfi_smp_create(device, ctypes.byref(self._ctx))
        if rc:
            raise SamplerError(f"bfi_smp_create: {self._L.bfi_smp_last_error(None).decode()}")
        self.device = device

    def close(self):
        if self._ctx:
            self._L.bfi_smp_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc:
            raise SamplerError(f"{what} (status {rc}): {self._L.bfi_smp_last_error(self._ctx).decode()}")

    @staticmethod
    def _stream(stream):
        if stream is None:
            import torch

            return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        return ctypes.c_void_p(stream)

    def set_tracing(self, on: bool):
        self._check(self._L.bfi_smp_set_tracing(self._ctx, 1 if on else 0), "bfi_smp_set_tracing")

    def trace(self, max_words=1 << 22):
        out = np.zeros(max_words, np.uint64)
        n = self._L.bfi_smp_trace(self._ctx, _np_ptr(out), max_words)
        if n < 0:
            raise SamplerError("bfi_smp_trace failed")
        return out[:n]

    def set_profiling(self, on: bool):
        self._check(self._L.bfi_smp_set_profiling(self._ctx, 1 if on else 0), "bfi_smp_set_profiling")

    def profile(self):
        """({k_stream, k_quant, k_row, call}: ms, launches) summed over the launches since the
        last call ("call": k_stream's start to k_row's end, gaps included)."""
        ms = (ctypes.c_double * 4)()
        n = ctypes.c_int64(0)
        self._check(self._L.bfi_smp_profile(self._ctx, ms, ctypes.byref(n)), "bfi_smp_profile")
        return {"k_stream": ms[0], "k_quant": ms[1], "k_row": ms[2], "call": ms[3]}, n.value

    def sample_rows(self, logits, params, u, out, hist=None, hist_off=None, mask=None, stream=None):
        """logits: cuda [B, V] float32 or bfloat16; params: cuda uint8 [B*32]; u: cuda f32 [B];
        out: cuda int32 [B]; hist: cuda int32 ids; hist_off: cuda int64 [B+1]; mask: cuda int32 [B, W]."""
        import torch

        B, V = logits.shape
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        ms = 0 if mask is None else mask.stride(0)
        rc = self._L.bfi_smp_sample_rows(self._ctx, _dptr(logits), dtype, B, V, logits.stride(0), _dptr(params),
                                         _dptr(hist), _dptr(hist_off), _dptr(mask), ms, _dptr(u), _dptr(out),
                                         self._stream(stream))
        self._check(rc, "bfi_smp_sample_rows")
        return out

    def head(self, x, norm_w, eps, w, out=None, norm_per_row=False, stream=None):
        """The output head on the device (qwen3.rs:258-265): rms_norm then lm_head over f32
        weights, bit-identical to the reference's CPU backend. x: cuda f32 [T, d]; norm_w:
        [d] (or [T, d]); w: [V, d]; returns the [T, V] f32 logits."""
        import torch

        T, d = x.shape
        V = w.shape[0]
        if out is None:
            out = torch.empty((T, V), dtype=torch.float32, device=x.device)
        rc = self._L.bfi_smp_head(self._ctx, _dptr(x), _dptr(norm_w), 1 if norm_per_row else 0, ctypes.c_float(eps),
                                  _dptr(w), T, d, V, _dptr(out), self._stream(stream))
        self._check(rc, "bfi_smp_head")
        return out

    def dequant(self, ggml_type, src, n_weights, out=None, stream=None):
        """A GGML tensor's weights (src: its bytes, a cuda uint8 tensor) to f32 on the device,
        each value as the reference's dequant_row computes it; returns the flat f32 tensor."""
        import torch

        if out is None:
            out = torch.empty(n_weights, dtype=torch.float32, device=src.device)
        rc = self._L.bfi_smp_dequant(self._ctx, int(ggml_type), _dptr(src), int(n_weights), _dptr(out),
                                     self._stream(stream))
        self._check(rc, "bfi_smp_dequant")
        return out

    def head_typed(self, x, norm_w, eps, w, ggml_type, out=None, norm_per_row=False, stream=None):
        """head over weights dequantized from GGML type ggml_type, in that type's dot order."""
        import torch

        T, d = x.shape
        V = w.shape[0]
        if out is None:
            out = torch.empty((T, V), dtype=torch.float32, device=x.device)
        rc = self._L.bfi_smp_head_typed(self._ctx, _dptr(x), _dptr(norm_w), 1 if norm_per_row else 0,
                                        ctypes.c_float(eps), _dptr(w), int(ggml_type), T, d, V, _dptr(out),
                                        self._stream(stream))
        self._check(rc, "bfi_smp_head_typed")
        return out

    def head_typed_sample_rows(self, x, norm_w, eps, w, ggml_type, params, u, out, hist=None, hist_off=None,
                               mask=None, norm_per_row=False, stream=None):
        """The fused device step over weights dequantized from GGML type ggml_type."""
        T, d = x.shape
        V = w.shape[0]
        ms = 0 if mask is None else mask.stride(0)
        rc = self._L.bfi_smp_head_typed_sample_rows(self._ctx, _dptr(x), _dptr(norm_w), 1 if norm_per_row else 0,
                                                    ctypes.c_float(eps), _dptr(w), int(ggml_type), T, d, V,
                                                    _dptr(params), _dptr(hist), _dptr(hist_off), _dptr(mask), ms,
                                                    _dptr(u), _dptr(out), self._stream(stream))
        self._check(rc, "bfi_smp_head_typed_sample_rows")
        return out

    def head_sample_rows(self, x, norm_w, eps, w, params, u, out, hist=None, hist_off=None, mask=None,
                         norm_per_row=False, stream=None):
        """The fused device step: head, then sample_rows over its logits; out: cuda int32 [T]."""
        T, d = x.shape
        V = w.shape[0]
        ms = 0 if mask is None else mask.stride(0)
        rc = self._L.bfi_smp_head_sample_rows(self._ctx, _dptr(x), _dptr(norm_w), 1 if norm_per_row else 0,
                                              ctypes.c_float(eps), _dptr(w), T, d, V, _dptr(params), _dptr(hist),
                                              _dptr(hist_off), _dptr(mask), ms, _dptr(u), _dptr(out),
                                              self._stream(stream))
        self._check(rc, "bfi_smp_head_sample_rows")
        return out

    def sample_rows_noalloc(self, logits, params, u, out, hist=None, hist_off=None, mask=None, stream=None):
        """sample_rows in the library's fixed per-device workspace (bfi_smp_sample_rows_noalloc:
        no device allocation; calls that overlap on one GPU race)."""
        import torch

        B, V = logits.shape
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        ms = 0 if mask is None else mask.stride(0)
        rc = self._L.bfi_smp_sample_rows_noalloc(self._ctx, _dptr(logits), dtype, B, V, logits.stride(0),
                                                 _dptr(params), _dptr(hist), _dptr(hist_off), _dptr(mask), ms,
                                                 _dptr(u), _dptr(out), self._stream(stream))
        self._check(rc, "bfi_smp_sample_rows_noalloc")
        return out

    def target_rows(self, logits, params, u, cap, hist=None, hist_off=None, mask=None, stream=None):
        import torch

        B, V = logits.shape
        dev = logits.device
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        o = dict(
            token=torch.zeros(B, dtype=torch.int32, device=dev),
            kind=torch.full((B,), -1, dtype=torch.int32, device=dev),
            kept_len=torch.zeros(B, dtype=torch.int32, device=dev),
            listed=torch.zeros(B, dtype=torch.int32, device=dev),
            ids=torch.zeros((B, max(cap, 1)), dtype=torch.int32, device=dev),
            probs=torch.zeros((B, max(cap, 1)), dtype=torch.float32, device=dev),
            stats=torch.zeros((B, 4), dtype=torch.float32, device=dev),
        )
        ms = 0 if mask is None else mask.stride(0)
        rc = self._L.bfi_smp_target_rows(
            self._ctx, _dptr(logits), dtype, B, V, logits.stride(0), _dptr(params), _dptr(hist), _dptr(hist_off),
            _dptr(mask), ms, _dptr(u), _dptr(o["token"]), _dptr(o["kind"]), _dptr(o["kept_len"]),
            _dptr(o["listed"]), _dptr(o["ids"]), _dptr(o["probs"]), cap, _dptr(o["stats"]), self._stream(stream))
        self._check(rc, "bfi_smp_target_rows")
        return o

    def verify(self, logits, rows_per_seq, params, drafts, draft_len, u_pairs, u_bonus, out_accepted, out_next,
               hist=None, hist_off=None, mask=None, stream=None):
        """logits: cuda [n_seq*rows_per_seq, V]; params per sequence; drafts [n_seq, rows_per_seq-1]."""
        import torch

        R, V = logits.shape
        n_seq = R // rows_per_seq
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        ms = 0 if mask is None else mask.stride(0)
        rc = self._L.bfi_smp_verify(
            self._ctx, _dptr(logits), dtype, n_seq, rows_per_seq, V, logits.stride(0), _dptr(params), _dptr(hist),
            _dptr(hist_off), _dptr(drafts), _dptr(draft_len), _dptr(mask), ms, _dptr(u_pairs), _dptr(u_bonus),
            _dptr(out_accepted), _dptr(out_next), self._stream(stream))
        self._check(rc, "bfi_smp_verify")

    def sample(self, logits, prev, params: dict, mask=None, u: float = 0.0) -> int:
        """`sample(logits, prev, &SampleParams)` (sample.rs:304) for one host row."""
        x = np.ascontiguousarray(logits, dtype=np.float32)
        h = np.ascontiguousarray(prev, dtype=np.uint32)
        p = params_array(params)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
        tok = ctypes.c_uint32(0)
        rc = self._L.bfi_smp_sample_host(self._ctx, _np_ptr(x), x.size, _np_ptr(h), h.size, _np_ptr(p), _np_ptr(m),
                                         u, ctypes.byref(tok))
        self._check(rc, "bfi_smp_sample_host")
        return tok.value

    def sample_seeded(self, logits, prev, params: dict, seed: int = 0, mask=None) -> int:
        """Exactly the reference call: u = Rng(seed).f32() (sample.rs:307)."""
        u, _ = rng_f32(seed)
        return self.sample(logits, prev, params, mask, u)


class MaskProducer:
    """Allow-mask producer of the decode-based constraint (apply_constraint, sample.rs:63-90)
    over a vocabulary of decoded pieces held on the GPU."""

    def __init__(self, device: int = 0):
        L = lib()
        h = ctypes.c_void_p()
        rc = L.bfi_mask_create(device, ctypes.byref(h))
        if rc != 0:
            raise SamplerError(f"bfi_mask_create failed ({rc})")
        self._h = h
        self.V = None

    def _check(self, rc):
        if rc != 0:
            raise SamplerError(lib().bfi_mask_error(self._h).decode(errors="replace"))

    def set_vocab(self, pieces):
        """pieces: list of bytes, piece i = decode(i)."""
        off = np.zeros(len(pieces) + 1, np.int64)
        off[1:] = np.cumsum([len(x) for x in pieces])
        blob = np.frombuffer(b"".join(pieces) or b"\0", np.uint8).copy()
        self._check(lib().bfi_mask_set_vocab(self._h, _np_ptr(blob), _np_ptr(off), len(pieces)))
        self.V = len(pieces)

    def build(self, so_far: bytes, d_mask, json_object=False, tool_choice=TOOL_NONE, tool_name=b"",
              tool_names=(), grammar=None, stream=None):
        """Writes the packed allow-mask into d_mask (torch uint32-compatible int32 tensor of
        ceil(V/32) words on the GPU); returns 0 when nothing is constrained, else 1."""
        g = None if grammar is None else (grammar.encode() if isinstance(grammar, str) else bytes(grammar))
        key = (bool(json_object), int(tool_choice), bytes(tool_name), tuple(bytes(n) for n in tool_names), g)
        cached = self._prepared.get(key) if hasattr(self, "_prepared") else None
        if cached is None:  # the constraint struct and the arrays it points into, kept per key
            keep = []

            def buf(b):
                a = np.frombuffer(b or b"\0", np.uint8).copy()
                keep.append(a)
                return _np_ptr(a)

            names = list(key[3])
            name_ptrs = (ctypes.c_void_p * max(len(names), 1))(*[buf(n) for n in names])
            name_lens = np.array([len(n) for n in names] or [0], np.int64)
            keep += [name_ptrs, name_lens]
            c = Constraint(int(key[0]), key[1], buf(key[2]), len(key[2]), ctypes.cast(name_ptrs, ctypes.c_void_p),
                           _np_ptr(name_lens), len(names), None if g is None else buf(g), 0 if g is None else len(g))
            if not hasattr(self, "_prepared") or len(self._prepared) > 64:
                self._prepared = {}
            cached = self._prepared[key] = (c, keep)
        c = cached[0]
        sf = np.frombuffer(so_far or b"\0", np.uint8)
        flag = ctypes.c_int32(-1)
        if stream is None:
            import torch

            stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self._check(lib().bfi_mask_build(self._h, _np_ptr(sf), len(so_far), ctypes.byref(c), _dptr(d_mask),
                                         ctypes.byref(flag), stream))
        return flag.value

    def close(self):
        if self._h:
            lib().bfi_mask_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- prefix cache (include/bfi_prefix.h; engine/prefix.rs) ---------------------------------


def _addr(a):
    """Address of a numpy array (host cache) or a torch tensor (device cache)."""
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        assert a.flags.c_contiguous
        return a.ctypes.data
    assert a.is_contiguous()
    return a.data_ptr()


def _nbytes(a):
    return a.nbytes if isinstance(a, np.ndarray) else a.numel() * a.element_size()


class PrefixCache:
    """PrefixCache (engine/prefix.rs:114-347) over the C ABI. device=-1 keeps entries in host
    memory (numpy arrays in and out), device>=0 in that GPU's memory (torch tensors on it).

    A state is (n, kv, rec, logits): kv a list of tensors whose first dimension is the
    position (their first n rows are kept), or whole tensors (indices in `whole`); rec a list
    of recurrent tensors or None per layer; logits a float32 vector."""

    def __init__(self, budget_bytes: int, device: int = -1):
        self._L = lib()
        self._pc = ctypes.c_void_p()
        rc = self._L.bfi_pc_create(device, budget_bytes, ctypes.byref(self._pc))
        if rc != 0:
            raise SamplerError(f"bfi_pc_create({device}) failed: {rc}")
        self.device = device

    def close(self):
        if self._pc:
            self._L.bfi_pc_destroy(self._pc)
            self._pc = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc != 0:
            raise SamplerError(f"{what}: {self._L.bfi_pc_last_error(self._pc).decode()} (status {rc})")

    @staticmethod
    def _state(n, kv, rec, logits, whole=()):
        ts = (PCTensor * max(len(kv), 1))()
        for i, t in enumerate(kv):
            if i in whole:
                ts[i] = PCTensor(_addr(t), 0, _nbytes(t))
            else:
                rows = t.shape[0]
                ts[i] = PCTensor(_addr(t), _nbytes(t) // rows if rows else 0, rows)
        rs = (PCTensor * max(len(rec), 1))()
        for i, t in enumerate(rec):
            rs[i] = PCTensor(None, 0, 0) if t is None else PCTensor(_addr(t), 0, _nbytes(t))
        nl = 0 if logits is None else (logits.size if isinstance(logits, np.ndarray) else logits.numel())
        st = PCState(n, ctypes.cast(ts, ctypes.c_void_p), len(kv), ctypes.cast(rs, ctypes.c_void_p), len(rec),
                     _addr(logits), nl)
        return st, (ts, rs)

    def lookup(self, ids):
        """prefix.rs:168-214: (id, matched, restore) or None."""
        a = np.ascontiguousarray(np.asarray(ids, np.uint32))
        hit, found = PCHit(), ctypes.c_int32(0)
        self._check(self._L.bfi_pc_lookup(self._pc, _np_ptr(a), a.size, ctypes.byref(hit), ctypes.byref(found)),
                    "bfi_pc_lookup")
        return (hit.id, hit.matched, hit.restore) if found.value else None

    def prepare(self, n, kv, rec, logits, whole=()):
        """The C description of a state, built once for calls that reuse the same tensors."""
        return self._state(n, kv, rec, logits, whole)

    def restore(self, hit, kv=None, rec=None, logits=None, whole=(), stream=None, prepared=None):
        """prefix.rs:217-230 into the given full-capacity tensors: (n, logits_restored) or None."""
        st, keep = prepared if prepared is not None else self._state(0, kv, rec, logits, whole)
        h = PCHit(*hit)
        n, lr, found = ctypes.c_uint64(0), ctypes.c_int32(0), ctypes.c_int32(0)
        self._check(self._L.bfi_pc_restore(self._pc, ctypes.byref(h), ctypes.byref(st), ctypes.byref(n),
                                           ctypes.byref(lr), ctypes.byref(found), stream), "bfi_pc_restore")
        return (n.value, bool(lr.value)) if found.value else None

    def insert(self, tokens, n=None, kv=None, rec=None, logits=None, whole=(), stream=None, prepared=None):
        """prefix.rs:233-260 (insert_copy / insert_owned)."""
        a = np.ascontiguousarray(np.asarray(tokens, np.uint32))
        st, keep = prepared if prepared is not None else self._state(n, kv, rec, logits, whole)
        self._check(self._L.bfi_pc_insert(self._pc, _np_ptr(a), a.size, ctypes.byref(st), stream), "bfi_pc_insert")

    def used_bytes(self):
        return self._L.bfi_pc_used_bytes(self._pc)

    def __len__(self):
        return self._L.bfi_pc_len(self._pc)

    def note_forward(self, n):
        self._L.bfi_pc_note_forward(self._pc, n)

    def forwarded(self):
        return self._L.bfi_pc_forwarded(self._pc)

    def clear(self):
        self._L.bfi_pc_clear(self._pc)
