"""Pins of the oracle's output head (oracle/bfi_oracle.c orc_rms_norm / orc_matmul_f32,
restating crates/bfi-core/src/cpu.rs:92-120 and 498-514): the reference's own KATs
(cpu.rs:835-855) and an independent statement of the rounding, numpy's float32 accumulate
(one rounded addition at a time, in order) with float32 products and numpy's correctly rounded
float32 sqrt. A dropped term, a reordered sum, a fused multiply-add or a sum from +0.0 fails
one of them."""
import numpy as np

import oracle as O


def test_reference_kats():
    # cpu.rs:835-842 rms_norm_ones: ones normalize to ones (exactly, in f32)
    y = O.rms_norm(np.ones((2, 3), np.float32), np.ones(3, np.float32), 0.0)
    assert (y == 1.0).all()
    # cpu.rs:844-855 matmul_f32_identity
    w = np.eye(3, dtype=np.float32)
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    assert O.matmul_f32(w, x).tolist() == [[1, 2, 3], [4, 5, 6]]


def _np_dot(a, b):
    p = (a.astype(np.float32) * b.astype(np.float32)).astype(np.float32)
    return np.add.accumulate(p, dtype=np.float32)[-1] if p.size else np.float32(-0.0)


def test_matmul_matches_sequential_float32_sums():
    rng = np.random.default_rng(0)
    for n_in in (1, 3, 16, 17, 255, 1024):
        w = (rng.standard_normal((9, n_in)) * rng.choice([1e-3, 1.0, 1e3], (9, 1))).astype(np.float32)
        x = rng.standard_normal((4, n_in)).astype(np.float32)
        got = O.matmul_f32(w, x)
        want = np.array([[_np_dot(w[o], x[t]) for o in range(9)] for t in range(4)], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n_in
    # the order matters: a pairwise or reversed sum of these terms rounds differently
    w = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    x = np.ones((1, 4), np.float32)
    assert O.matmul_f32(w, x)[0, 0] == np.float32(1.0)  # ((1e8 + 1) - 1e8) + 1 = 0 + 1
    # an all-zero dot keeps the sign of zero a sum from -0.0 gives
    assert np.signbit(O.matmul_f32(np.array([[-0.0, 0.0]], np.float32), np.array([[1.0, -1.0]], np.float32))[0, 0])


def test_rms_norm_matches_numpy_statement():
    rng = np.random.default_rng(1)
    for d in (1, 5, 64, 1000, 4096):
        x = (rng.standard_normal((3, d)) * rng.choice([1e-20, 1e-3, 1.0, 1e15], (3, 1))).astype(np.float32)
        w = rng.standard_normal(d).astype(np.float32)
        for eps in (0.0, 1e-6):
            got = O.rms_norm(x, w, eps)
            for r in range(3):
                s = np.add.accumulate((x[r] * x[r]).astype(np.float32), dtype=np.float32)[-1]
                mean = np.float32(s / np.float32(d))
                scale = np.float32(np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(eps))))
                want = ((x[r] * scale).astype(np.float32) * w).astype(np.float32)
                assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), (d, eps, r)
    # per-row weights
    x = rng.standard_normal((2, 8)).astype(np.float32)
    w2 = rng.standard_normal((2, 8)).astype(np.float32)
    got = O.rms_norm(x, w2, 1e-5, w_per_row=True)
    assert np.array_equal(got[1], O.rms_norm(x[1:], w2[1], 1e-5)[0])
