"""GPU parity of the output head (bfi_smp_head, include/bfi_sampler.h): the device logits equal
the oracle's restatement of the reference's CPU head (rms_norm + matmul_f32, cpu.rs:92-120,
498-514) bit for bit, at odd and unaligned shapes and at a Qwen3-0.6B-sized head
(n_embd 1024, n_vocab 151936); and the fused head + sample step draws the oracle's tokens."""
import numpy as np
import pytest

import bfi_smp
import oracle as O
import workloads

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def smp(gpu):
    s = bfi_smp.Sampler(0)
    yield s
    s.close()


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _case(rng, T, d, V, scale=1.0, per_row=False):
    x = (rng.standard_normal((T, d)) * scale).astype(np.float32)
    nw = rng.standard_normal((T, d) if per_row else d).astype(np.float32)
    w = (rng.standard_normal((V, d)) / np.sqrt(d)).astype(np.float32)
    return x, nw, w


@pytest.mark.parametrize("T,d,V,per_row", [(1, 1, 1, False), (3, 5, 7, False), (2, 17, 130, True), (70, 64, 65, False),
                                           (5, 130, 1000, False), (64, 256, 4099, True)])
def test_head_matches_oracle_bitwise(smp, T, d, V, per_row):
    import torch

    rng = np.random.default_rng(T * 1000 + d)
    x, nw, w = _case(rng, T, d, V, scale=float(rng.choice([1e-3, 1.0, 30.0])), per_row=per_row)
    got = smp.head(_dev(x), _dev(nw), 1e-6, _dev(w), norm_per_row=per_row)
    torch.cuda.synchronize()
    want = O.matmul_f32(w, O.rms_norm(x, nw, 1e-6, w_per_row=per_row))
    g = got.cpu().numpy()
    bad = np.nonzero(g.view(np.uint32) != want.view(np.uint32))
    assert bad[0].size == 0, (T, d, V, bad[0][:5], bad[1][:5])


def test_head_unaligned_weights(smp):
    """Weights starting 4 bytes into an allocation take the scalar loads."""
    import torch

    rng = np.random.default_rng(5)
    x, nw, w = _case(rng, 4, 64, 300)
    big = torch.empty(w.size + 1, dtype=torch.float32, device="cuda:0")
    big[1:] = _dev(w.reshape(-1))
    wv = big[1:].view(300, 64)
    got = smp.head(_dev(x), _dev(nw), 1e-5, wv)
    torch.cuda.synchronize()
    want = O.matmul_f32(w, O.rms_norm(x, nw, 1e-5))
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_qwen3_sized_head_and_fused_sampling(smp):
    """n_embd 1024, n_vocab 151936, 4 rows (the oracle's head takes ~1 s a row): logits equal
    bit for bit, and head_sample_rows draws the tokens the oracle samples from those logits."""
    import torch

    rng = np.random.default_rng(9)
    T, d, V = 4, 1024, 151936
    x, nw, w = _case(rng, T, d, V, scale=3.0)
    w *= 8.0  # peaked rows: a few ids far above the rest
    xd, nwd, wd = _dev(x), _dev(nw), _dev(w)
    got = smp.head(xd, nwd, 1e-6, wd)
    torch.cuda.synchronize()
    logits = O.matmul_f32(w, O.rms_norm(x, nw, 1e-6))
    assert np.array_equal(got.cpu().numpy().view(np.uint32), logits.view(np.uint32))
    rows = [dict(temperature=0.8, top_p=0.95), dict(temperature=0.0), dict(temperature=1.0, top_k=40, min_p=0.05),
            dict(temperature=0.6, top_p=0.9, repeat_penalty=1.1)]
    params = bfi_smp.params_array(rows)
    hist = rng.integers(0, V, 32).astype(np.uint32)
    off = np.array([0, 8, 16, 24, 32], np.int64)
    u = rng.random(T).astype(np.float32)
    out = torch.zeros(T, dtype=torch.int32, device="cuda:0")
    pd = torch.from_numpy(params.view(np.uint8)).to("cuda:0")
    smp.head_sample_rows(xd, nwd, 1e-6, wd, pd, _dev(u), out, _dev(hist.view(np.int32)), _dev(off))
    torch.cuda.synchronize()
    want = O.sample_rows(logits, params, hist, off, u)
    assert out.cpu().numpy().astype(np.uint32).tolist() == [int(t) for t in want]


# ---- quantized lm_head weights (bfi_smp_dequant, bfi_smp_head_typed) ---------------------------

BLOCK = {1: (1, 2), 30: (1, 2), 8: (32, 34), 2: (32, 18), 14: (256, 210), 12: (256, 144), 13: (256, 176), 41: (128, 18),
         142: (128, 34), 143: (128, 28)}


def _random_tensor(rng, ggml_type, n):
    """Random bytes of a GGML tensor of n weights with finite f16 scales."""
    be, bb = BLOCK[ggml_type]
    nb = n // be
    raw = rng.integers(0, 256, nb * bb, dtype=np.uint8).reshape(nb, bb)
    if ggml_type == 1:  # finite f16 weights
        raw = (rng.standard_normal(n) * 0.1).astype(np.float16).view(np.uint8).reshape(nb, bb)
    elif ggml_type == 30:  # finite bf16 weights (the top halves of f32 values)
        top = ((rng.standard_normal(n) * 0.1).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        raw = top.view(np.uint8).reshape(nb, bb)
    elif ggml_type in (8, 2):
        raw[:, 0:2] = (rng.standard_normal(nb) * 0.01).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif ggml_type in (41, 142):
        raw[:, 0:2] = (rng.standard_normal(nb) * 0.01).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif ggml_type == 143:
        raw[:, 26:28] = (rng.standard_normal(nb) * 0.01).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif ggml_type == 14:
        raw[:, 208:210] = (rng.standard_normal(nb) * 0.001).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif ggml_type in (12, 13):  # d and dmin
        raw[:, 0:4] = (rng.standard_normal(2 * nb) * 0.001).astype(np.float16).view(np.uint8).reshape(nb, 4)
    return raw.reshape(-1)


@pytest.mark.parametrize("ggml_type", [1, 30, 8, 2, 14, 12, 13, 41, 142, 143])
def test_device_dequant_matches_oracle(smp, ggml_type):
    import torch

    rng = np.random.default_rng(ggml_type)
    n = 256 * 97
    src = _random_tensor(rng, ggml_type, n)
    got = smp.dequant(ggml_type, _dev(src), n)
    torch.cuda.synchronize()
    want = O.dequant(ggml_type, src, n)
    g = got.cpu().numpy()
    fin = np.isfinite(want)
    assert np.array_equal(g[fin].view(np.uint32), want[fin].view(np.uint32))
    assert (np.isnan(g) == np.isnan(want)).all()


@pytest.mark.parametrize("ggml_type,d", [(8, 256), (8, 1000), (2, 64), (14, 256), (12, 512), (13, 256), (1, 130),
                                         (30, 64), (41, 256), (41, 224), (142, 384), (143, 256), (143, 96)])
def test_typed_head_matches_oracle_bitwise(smp, ggml_type, d):
    """Q8_0 / Q4_0 (PQ2_0 / PTQ1_0) rows of whole blocks take the 32- (128-) weight block dot
    order, Q1_0 rows of whole blocks its signed blocks, other rows one dot."""
    import torch

    rng = np.random.default_rng(ggml_type * 7 + d)
    T, V = 9, 1028
    x = rng.standard_normal((T, d)).astype(np.float32)
    nw = rng.standard_normal(d).astype(np.float32)
    src = _random_tensor(rng, ggml_type, V * d)
    w_dev = smp.dequant(ggml_type, _dev(src), V * d).view(V, d)
    out = smp.head_typed(_dev(x), _dev(nw), 1e-6, w_dev, ggml_type)
    torch.cuda.synchronize()
    w = O.dequant(ggml_type, src, V * d).reshape(V, d)
    xn = O.rms_norm(x, nw, 1e-6)
    block = 32 if ggml_type in (8, 2) and d % 32 == 0 else 128 if ggml_type in (142, 143) and d % 128 == 0 else 0
    if ggml_type == 41 and d % 128 == 0:
        block = 128
        want = O.matmul_signs(w, xn, 128)
    else:
        want = O.matmul_blocked(w, xn, block)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    if block:  # the order matters at this size: the one-dot order differs somewhere
        assert not np.array_equal(O.matmul_f32(w, xn).view(np.uint32), want.view(np.uint32))


def test_dequant_rejects_partial_blocks_and_other_types(smp):
    import torch

    src = torch.zeros(64, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(bfi_smp.SamplerError):
        smp.dequant(8, src, 31)
    with pytest.raises(bfi_smp.SamplerError):
        smp.dequant(6, src, 32)  # Q5_0: not taken
    with pytest.raises(bfi_smp.SamplerError):
        smp.dequant(143, src, 64)  # PTQ1_0: half a block


def test_typed_fused_step_draws_the_oracles_tokens(smp):
    """A Q8_0 lm_head (n_embd 256, 20,000 ids): head_typed_sample_rows draws the tokens the oracle
    samples from the oracle's block-order logits."""
    import torch

    rng = np.random.default_rng(21)
    T, d, V = 4, 256, 20000
    x = (rng.standard_normal((T, d)) * 3).astype(np.float32)
    nw = rng.standard_normal(d).astype(np.float32)
    src = _random_tensor(rng, 8, V * d)
    src.reshape(-1, 34)[:, 0:2] = (np.abs(rng.standard_normal(V * d // 32)) * 0.05 + 0.01).astype(
        np.float16).view(np.uint8).reshape(-1, 2)  # (peaked rows)
    wd = smp.dequant(8, _dev(src), V * d).view(V, d)
    w = O.dequant(8, src, V * d).reshape(V, d)
    logits = O.matmul_blocked(w, O.rms_norm(x, nw, 1e-6), 32)
    rows = [dict(temperature=0.8, top_p=0.95), dict(temperature=0.0), dict(temperature=1.0, top_k=40, min_p=0.05),
            dict(temperature=0.6, top_p=0.9, repeat_penalty=1.1)]
    params = bfi_smp.params_array(rows)
    hist = rng.integers(0, V, 32).astype(np.uint32)
    off = np.array([0, 8, 16, 24, 32], np.int64)
    u = rng.random(T).astype(np.float32)
    out = torch.zeros(T, dtype=torch.int32, device="cuda:0")
    pd = torch.from_numpy(params.view(np.uint8)).to("cuda:0")
    smp.head_typed_sample_rows(_dev(x), _dev(nw), 1e-6, wd, 8, pd, _dev(u), out, _dev(hist.view(np.int32)), _dev(off))
    torch.cuda.synchronize()
    want = O.sample_rows(logits, params, hist, off, u)
    assert out.cpu().numpy().astype(np.uint32).tolist() == [int(t) for t in want]
