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


# ---- lm_head weight formats (orc_dequant, orc_matmul_blocked) ----------------------------------


def _f16_bytes(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def test_dequant_f16_every_code_and_bf16_against_torch():
    codes = np.arange(65536, dtype=np.uint16)
    got = O.dequant(1, codes.view(np.uint8), 65536).view(np.uint32)
    want = codes.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got, want)
    import torch

    rng = np.random.default_rng(5)
    bits = rng.integers(0, 65536, 4096, dtype=np.uint16)
    got = O.dequant(30, bits.view(np.uint8), bits.size)
    want = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert (np.isnan(got) == np.isnan(want)).all()


def test_dequant_reference_kats():
    # q8_0.rs:21-31 and types/mod.rs:310-317: d = 1, qs[0] = 5, qs[1] = -3
    b = np.zeros(34, np.uint8)
    b[0:2] = _f16_bytes(1.0)
    b[2], b[3] = 5, np.uint8(256 - 3)
    out = O.dequant(8, b, 32)
    assert out[0] == 5.0 and out[1] == -3.0 and (out[2:] == 0).all()
    # q4_0.rs:24-32: d = 1, every nibble 0 -> -8
    b = np.zeros(18, np.uint8)
    b[0:2] = _f16_bytes(1.0)
    assert (O.dequant(2, b, 32) == -8.0).all()
    # q6_k.rs:36-41, types/mod.rs:324-327: an all-zero block (d = 0) is all zeros
    assert (O.dequant(14, np.zeros(210, np.uint8), 256) == 0.0).all()


def test_dequant_layouts_place_every_weight():
    """Blocks built by an encoder (the inverse of each layout) from known small-integer values:
    a wrong nibble, high-bit pair or scale index moves a value and fails."""
    # Q8_0: d = 0.5, q_i = i - 16
    b = np.zeros(34, np.uint8)
    b[0:2] = _f16_bytes(0.5)
    b[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    assert O.dequant(8, b, 32).tolist() == [(i - 16) * 0.5 for i in range(32)]
    # Q4_0: d = 2, weight j < 16 in the low nibble of byte j, weight j + 16 in its high nibble
    nib = np.arange(32) % 16
    nib[16:] = 15 - nib[16:]
    b = np.zeros(18, np.uint8)
    b[0:2] = _f16_bytes(2.0)
    b[2:] = (nib[:16] | (nib[16:] << 4)).astype(np.uint8)
    assert O.dequant(2, b, 32).tolist() == [float((v - 8) * 2) for v in nib]
    # Q6_K: d = 0.25, sixteen scales 1..16 (scale i covers weights 16 i .. 16 i + 15), and
    # q = (k * 7) % 64 - 32 at weight k, encoded into ql / qh
    q = (np.arange(256) * 7) % 64
    sc = np.arange(1, 17, dtype=np.int8)
    blk = np.zeros(210, np.uint8)
    for k in range(256):
        half, r = divmod(k, 128)
        quarter, l = divmod(r, 32)
        v = int(q[k])
        qi = half * 64 + l + (32 if quarter in (1, 3) else 0)
        blk[qi] |= (v & 15) << (4 if quarter >= 2 else 0)
        blk[128 + half * 32 + l] |= (v >> 4) << (2 * quarter)
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = _f16_bytes(0.25)
    # the scale of weight k: sixteen weights a scale, in the order the quarters are stored
    want = []
    for k in range(256):
        half, r = divmod(k, 128)
        quarter, l = divmod(r, 32)
        s = int(sc[half * 8 + l // 16 + 2 * quarter])
        want.append(0.25 * s * (int(q[k]) - 32))
    assert O.dequant(14, blk, 256).tolist() == want


def test_blocked_dot_keeps_what_one_row_sum_loses():
    w = np.array([[2.0 ** 24] + [1.0] * 63], np.float32)
    x = np.ones((1, 64), np.float32)
    assert O.matmul_blocked(w, x, 32)[0, 0] == 2.0 ** 24 + 32
    assert O.matmul_blocked(w, x, 0)[0, 0] == 2.0 ** 24
    # a partial last block sums what it holds
    w2 = np.array([[1.0] * 40], np.float32)
    assert O.matmul_blocked(w2, np.ones((1, 40), np.float32), 32)[0, 0] == 40.0


def _pack_scale_min_k4(sc, mn):
    """12 bytes holding eight 6-bit scales and mins, the inverse of get_scale_min_k4
    (k_scale.rs:3-11): sub-blocks 0-3 in the low 6 bits of bytes 0-7, sub-blocks 4-7 split
    into low nibbles (bytes 8-11) and top two bits (the high bits of bytes 0-7)."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return q


def test_dequant_k_quants_place_every_weight():
    """Q4_K and Q5_K blocks from an encoder: d = 0.5, dmin = 0.25, scales and mins 1..63 spread
    over all eight sub-blocks (so the packed high bits matter), nibble k % 16 at weight k and,
    for Q5_K, the high bit set on every third weight; the reference's all-zero KAT."""
    assert (O.dequant(12, np.zeros(144, np.uint8), 256) == 0.0).all()  # types/mod.rs:319-322
    sc = np.array([1, 7, 33, 63, 18, 45, 60, 5])
    mn = np.array([2, 62, 17, 9, 48, 31, 3, 40])
    for t, bb in ((12, 144), (13, 176)):
        blk = np.zeros(bb, np.uint8)
        blk[0:2] = _f16_bytes(0.5)
        blk[2:4] = _f16_bytes(0.25)
        blk[4:16] = _pack_scale_min_k4(sc, mn)
        qs = 16 if t == 12 else 48
        want = []
        for k in range(256):
            group, r = divmod(k, 64)
            hi, l = divmod(r, 32)
            nib = k % 16
            blk[qs + group * 32 + l] |= nib << (4 * hi)
            extra = 0
            if t == 13 and k % 3 == 0:
                blk[16 + l] |= 1 << (2 * group + hi)
                extra = 16
            j = 2 * group + hi
            want.append(np.float32(np.float32(0.5 * sc[j]) * np.float32(nib + extra)) - np.float32(0.25 * mn[j]))
        got = O.dequant(t, blk, 256)
        assert np.array_equal(got, np.array(want, np.float32)), t


def _f16(v):
    return np.array([v], np.float16).view(np.uint8)


def test_dequant_one_bit_and_ternary_reference_kats():
    # q1_0.rs tests: all clear is -d, all set +d; sign bits LSB first
    blk = np.concatenate([_f16(0.5), np.zeros(16, np.uint8)])
    assert (O.dequant(41, blk, 128) == -0.5).all()
    blk[2:] = 0xFF
    assert (O.dequant(41, blk, 128) == 0.5).all()
    blk = np.concatenate([_f16(2.0), np.zeros(16, np.uint8)])
    blk[2], blk[17] = 0b0000_0101, 0b1000_0000
    out = O.dequant(41, blk, 128)
    assert out[0] == 2.0 and out[1] == -2.0 and out[2] == 2.0 and out[126] == -2.0 and out[127] == 2.0
    # ptq1_0.rs tests: zero digits everywhere are -d
    blk = np.concatenate([np.zeros(26, np.uint8), _f16(2.0)])
    assert (O.dequant(143, blk, 128) == -2.0).all()


def test_dequant_pq2_0_places_every_code():
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 4, (3, 128))
    raw = np.zeros((3, 34), np.uint8)
    for b in range(3):
        raw[b, 0:2] = _f16(0.25 * (b + 1))
        for j in range(128):
            raw[b, 2 + j // 4] |= codes[b, j] << (2 * (j % 4))
    want = ((codes - 1) * (0.25 * (np.arange(3)[:, None] + 1))).astype(np.float32).reshape(-1)
    assert np.array_equal(O.dequant(142, raw.reshape(-1), 384), want)


def _tq_byte(trits):
    """The base-3 packing the digit reader inverts: the five digits as a fraction of 243 scaled
    to a byte, rounded up, so that digit n is the top base-3 digit of byte * 3^n mod 256."""
    q = 0
    for t in trits:
        q = q * 3 + int(t)
    return (q * 256 + 242) // 243


def test_dequant_ptq1_0_places_every_trit():
    # every 5-digit byte decodes back to its digits
    for q in range(243):
        digits = [(q // 3 ** (4 - n)) % 3 for n in range(5)]
        blk = np.zeros(28, np.uint8)
        blk[0] = _tq_byte(digits)
        blk[26:28] = _f16(1.0)
        out = O.dequant(143, blk, 128)
        assert [int(out[16 * n]) + 1 for n in range(5)] == digits
    # the layout: weights 0..79 digit j/16 of qs[j%16], 80..119 digit (j-80)/8 of qs[16+(j-80)%8],
    # 120..127 digit (j-120)/2 of qh[(j-120)%2] (ptq1_0.rs:15-24)
    rng = np.random.default_rng(11)
    t = rng.integers(0, 3, 128)
    dig = {}
    for j in range(128):
        at, n = (j % 16, j // 16) if j < 80 else (16 + (j - 80) % 8, (j - 80) // 8) if j < 120 else (24 + (j - 120) % 2, (j - 120) // 2)
        dig.setdefault(at, [0] * 5)[n] = t[j]
    blk = np.zeros(28, np.uint8)
    for at, ds in dig.items():
        blk[at] = _tq_byte(ds)
    blk[26:28] = _f16(0.5)
    assert np.array_equal(O.dequant(143, blk, 128), ((t - 1) * 0.5).astype(np.float32))


def test_signed_block_dot_scales_after_the_sum():
    d = 3 * 2.0 ** -7  # exact in f16
    w = np.full((1, 128), d, np.float32)
    x = np.ones((1, 128), np.float32)
    x[0, 0] = 2.0 ** 24
    # the ones vanish into 2^24 before the scale; taken product first they would round up
    assert O.matmul_signs(w, x)[0, 0] == 2.0 ** 24 * d
    assert O.matmul_blocked(w, x, 128)[0, 0] > 2.0 ** 24 * d
    # each block its own scale, signs from the weights, blocks added in order
    w2 = np.concatenate([np.full(128, 1.0), np.full(128, -2.0)]).astype(np.float32)[None]
    assert O.matmul_signs(w2, np.ones((1, 256), np.float32))[0, 0] == 128.0 - 256.0

