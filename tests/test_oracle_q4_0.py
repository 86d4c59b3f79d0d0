"""Pins for the oracle's Q4_0 and bf16 restatements (CPU only).

Known answers come from the GGUF Q4_0 definition (fp16 LE scale, low nibble
= element j, high nibble = element j + 16, value d * (nibble - 8)) and from
IEEE 754 binary16 / bfloat16 rounding.  The C and numpy restatements are
written independently (ldexp decode vs numpy float16) and must agree."""
import numpy as np
import pytest

from oracle import q4_0 as oq
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16


def one_block(d: float, codes) -> np.ndarray:
    return oq.pack_blocks(np.array([[d]], dtype=np.float16),
                          np.asarray(codes, dtype=np.uint8).reshape(1, 1, 32))


def test_kat_unit_scale_codes():
    codes = np.arange(32) % 16
    w = oq.dequant_f32(one_block(1.0, codes), 1, 32)[0]
    np.testing.assert_array_equal(w, (codes - 8).astype(np.float32))


def test_kat_nibble_order():
    """byte 0 = 0x1F: element 0 = 15 - 8 = 7, element 16 = 1 - 8 = -7."""
    blk = np.zeros((1, 18), dtype=np.uint8)
    blk[0, 0:2] = np.array([1.0], dtype="<f2").view(np.uint8)
    blk[0, 2] = 0x1F
    blk[0, 3:] = 0x88
    q, s = oq.unpack(blk, 1, 32)
    assert q[0, 0] == 7 and q[0, 16] == -7
    assert np.all(q[0, 1:16] == 0) and np.all(q[0, 17:] == 0)
    qc, sc = oq.c_unpack(blk, 1, 32)
    np.testing.assert_array_equal(q, qc)
    assert s[0, 0] == 1.0 and sc[0, 0] == 1.0


@pytest.mark.parametrize("d,expect", [
    (-0.0, None), (2.0 ** -24, None), (65504.0, None), (np.inf, None), (-np.inf, None)])
def test_kat_special_scales(d, expect):
    codes = np.arange(32) % 16
    blk = one_block(d, codes)
    w = oq.dequant_f32(blk, 1, 32)[0]
    wc = oq.c_dequant_f32(blk, 1, 32)[0]
    with np.errstate(invalid="ignore"):
        ref = np.float32(d) * (codes - 8).astype(np.float32)
    np.testing.assert_array_equal(w, ref)
    np.testing.assert_array_equal(wc, ref)
    if d == 2.0 ** -24:  # fp16 subnormal times a small integer stays exact
        assert w[15] == 7 * 2.0 ** -24
    if np.isinf(d):  # inf * 0 is NaN at code 8
        assert np.isnan(w[8]) and np.isnan(wc[8])


def test_kat_nan_scale_propagates():
    blk = one_block(np.nan, np.arange(32) % 16)
    assert np.isnan(oq.dequant_f32(blk, 1, 32)).all()
    assert np.isnan(oq.c_dequant_f32(blk, 1, 32)).all()


def test_c_fp16_decode_matches_numpy_for_every_pattern():
    lib = oq.c_lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.oracle_f16_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    r = ref[::7]
    nan = np.isnan(r)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan], r[~nan])


@pytest.mark.parametrize("f,bits", [
    (1.0, 0x3F80), (1.00390625, 0x3F80),        # tie, even stays
    (1.01171875, 0x3F82),                        # tie, odd rounds up
    (1.0078125, 0x3F81), (-2.0, 0xC000),
    (3.3895313892515355e38, 0x7F7F),             # largest finite bf16
    (float(np.uint32(0x7F7F8000).view(np.float32)), 0x7F80),  # tie above it -> inf
    (float("inf"), 0x7F80), (1e-45, 0x0000),
])
def test_bf16_rne_known_answers(f, bits):
    assert int(f32_to_bf16_bits(np.float32([f]))[0]) == bits
    assert int(oq.c_lib().oracle_f32_to_bf16(f)) == bits


def test_bf16_nan_stays_nan():
    assert np.isnan(bf16_bits_to_f32(f32_to_bf16_bits(np.float32([np.nan])))[0])


def test_c_and_numpy_dequant_agree():
    blocks = oq.make_blocks(64, 512, seed=1)
    np.testing.assert_array_equal(oq.dequant_f32(blocks, 64, 512), oq.c_dequant_f32(blocks, 64, 512))
    np.testing.assert_array_equal(oq.dequant_bf16_bits(blocks, 64, 512),
                                  oq.c_dequant_bf16_bits(blocks, 64, 512))
    q, s = oq.unpack(blocks, 64, 512)
    qc, sc = oq.c_unpack(blocks, 64, 512)
    np.testing.assert_array_equal(q, qc)
    np.testing.assert_array_equal(s.view(np.uint16), sc.view(np.uint16))


def test_generator_recipe():
    blocks = oq.make_blocks(300, 2560, seed=2)
    q, s = oq.unpack(blocks, 300, 2560)
    assert q.min() == -8 and q.max() == 7
    assert np.all(s >= 0)
    assert abs(float(np.mean(s.astype(np.float64))) - 0.02 * np.sqrt(2 / np.pi)) < 5e-4


def test_gemv_f64_matches_brute_force():
    rng = np.random.default_rng(0)
    n, k = 16, 128
    blocks = oq.make_blocks(n, k, seed=4)
    x = f32_to_bf16_bits(rng.standard_normal(k).astype(np.float32))
    xf = bf16_bits_to_f32(x).astype(np.float64)
    q, s = oq.unpack(blocks, n, k)
    brute = np.zeros(n)
    for r in range(n):
        for j in range(k):
            brute[r] += float(s[r, j // 32]) * float(q[r, j]) * xf[j]
    np.testing.assert_allclose(oq.gemv_f64(x, blocks, n, k), brute, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oq.gemv_np_f64(xf, blocks, n, k), brute, rtol=1e-12, atol=1e-12)


def test_gemv_one_hot_and_linearity_and_zero_scale():
    n, k = 32, 256
    blocks = oq.make_blocks(n, k, seed=5)
    w = oq.dequant_f32(blocks, n, k)
    e = np.zeros(k, dtype=np.uint16)
    e[37] = 0x3F80
    np.testing.assert_array_equal(oq.gemv_f64(e, blocks, n, k), w[:, 37].astype(np.float64))
    rng = np.random.default_rng(1)
    a = f32_to_bf16_bits(rng.standard_normal(k).astype(np.float32))
    b = f32_to_bf16_bits(rng.standard_normal(k).astype(np.float32))
    a[::2] = 0  # disjoint supports make a + b exact in bf16
    b[1::2] = 0
    ab = a | b
    np.testing.assert_allclose(oq.gemv_f64(ab, blocks, n, k),
                               oq.gemv_f64(a, blocks, n, k) + oq.gemv_f64(b, blocks, n, k),
                               rtol=1e-12, atol=1e-9)
    zero = blocks.copy().reshape(n, k // 32, 18)
    zero[:, :, 0:2] = 0
    assert not oq.gemv_f64(a, zero.reshape(n, -1), n, k).any()


def test_gemv_bf16_weight_rounding_kat():
    """gemv_bf16w_bits rounds each weight d * q to bf16 before the product
    (sva/kernels/linear.py:87-100).  Rows of 8 blocks with x = 1: blocks 0-3
    hold q = +1 (nibble 9) at an fp16 scale d that is not a bf16 value, blocks
    4-7 hold q = -1 at d = 1 (exact), so the row sum is 128 * (bf16(d) - 1)
    with weight rounding and 128 * (d - 1) without.
      d = 1 + 3 * 2^-10: bf16(d) = 1         -> 0       (exact 0.375)
      d = 1 + 5 * 2^-10: bf16(d) = 1 + 2^-7  -> 1.0     (exact 0.625)
      d = 1 + 4 * 2^-10: a tie, to even = 1  -> 0       (exact 0.5)
      d = 1 + 2^-7 (bf16-exact)              -> 1.0     (exact 1.0)
    A GEMV that skipped the weight rounding, or rounded ties away from zero,
    gives different bits."""
    n, k = 4, 256
    scales = [1 + 3 * 2.0 ** -10, 1 + 5 * 2.0 ** -10, 1 + 4 * 2.0 ** -10, 1 + 2.0 ** -7]
    d = np.empty((n, 8), dtype=np.float16)
    codes = np.empty((n, 8, 32), dtype=np.uint8)
    for r, s in enumerate(scales):
        d[r, :4] = s
        d[r, 4:] = 1.0
        codes[r, :4] = 9
        codes[r, 4:] = 7
    assert all(float(np.float16(s)) == s for s in scales)  # fp16-exact scales
    blocks = oq.pack_blocks(d, codes)
    x = np.full(k, 0x3F80, dtype=np.uint16)  # 1.0
    got = bf16_bits_to_f32(oq.gemv_bf16w_bits(x, blocks, n, k))
    np.testing.assert_array_equal(got, np.float32([0.0, 1.0, 0.0, 1.0]))
    np.testing.assert_array_equal(oq.gemv_f64(x, blocks, n, k), [0.375, 0.625, 0.5, 1.0])


def test_gemv_bf16_weight_variant_close_to_exact():
    rng = np.random.default_rng(3)
    n, k = 64, 2560
    blocks = oq.make_blocks(n, k, seed=6)
    x = f32_to_bf16_bits(rng.standard_normal(k).astype(np.float32))
    exact = oq.gemv_f64(x, blocks, n, k)
    ref = bf16_bits_to_f32(oq.gemv_bf16w_bits(x, blocks, n, k))
    assert np.max(np.abs(ref - exact) / (np.abs(exact) + 0.05)) < 2e-2
    assert np.array_equal(round_bf16(np.float32([1.5])), np.float32([1.5]))


def _kat_blocks(rows: int) -> np.ndarray:
    """rows x 256 weights (8 blocks each), every byte distinct enough to place:
    scale bytes (0x10 + row, 0x40 + block), qs[j] = (row * 8 + block) * 16 + j
    (mod 256)."""
    blk = np.zeros((rows, 8, 18), dtype=np.uint8)
    for r in range(rows):
        for j in range(8):
            blk[r, j, 0], blk[r, j, 1] = 0x10 + r, 0x40 + j
            blk[r, j, 2:] = ((r * 8 + j) * 16 + np.arange(16)) % 256
    return blk.reshape(rows, -1)


def test_repack_known_bytes():
    """Literal bytes of the packed layout for a 2-row, 256-k matrix (one group,
    one chunk).  Row 1 block 7 has qs = 0xF0..0xFF: lane 16*2 + 1 (row 1,
    k-group 2), byte 1 of word 3 of the second half holds elements 17 and 21
    = high nibbles of qs[1] = 0xF1 and qs[5] = 0xF5 -> 0xFF; row 0 block 0
    (qs = 0x00..0x0F), lane 0 byte 0: elements 0 and 4 = low nibbles of qs[0]
    and qs[4] -> 0x40; lane 16*1 (k-group 1) byte 2: elements 10 and 14 ->
    0xEA.  Rows 2..15 of the group repeat row 1."""
    wp = oq.repack(_kat_blocks(2), 2, 256)
    assert wp.size == 2304 == oq.packed_bytes(2, 256)
    assert wp[1024 + 16 * (16 * 2 + 1) + 4 * 3 + 1] == 0xFF
    assert wp[0] == 0x40
    assert wp[16 * 16 + 2] == 0xEA
    # row 0, block 1 (qs 0x10..0x1F), k-group 3, byte 3: elements 27 and 31 =
    # high nibbles of qs[11] = 0x1B and qs[15] = 0x1F -> 0x11
    assert wp[16 * (16 * 3 + 0) + 4 * 1 + 3] == 0x11
    # padding row 9 repeats row 1 (block 7 byte as above)
    assert wp[1024 + 16 * (16 * 2 + 9) + 4 * 3 + 1] == 0xFF
    # scales: row 1, block 5 -> bytes (0x11, 0x45) at 2048 + 16 + 10
    assert (wp[2048 + 16 + 10], wp[2048 + 16 + 11]) == (0x11, 0x45)
    assert (wp[2048 + 16 * 15 + 14], wp[2048 + 16 * 15 + 15]) == (0x11, 0x47)


def test_repack_known_bytes_gated():
    """Gated, d = 3 (rows 0-2 gate, 3-5 up): lane row r < 8 is gate row
    min(r, 2), r >= 8 up row 3 + min(r - 8, 2).  Row 5 block 0 has qs = 0x80 +
    j: lane row 10, k-group 0, byte 0 -> elements 0, 4 = 0x0, 0x4 -> 0x40;
    its scale bytes are (0x15, 0x40)."""
    wp = oq.repack(_kat_blocks(6), 3, 256, gated=True)
    assert wp.size == 2304 == oq.packed_bytes(3, 256, gated=True)
    assert (wp[2048 + 16 * 10], wp[2048 + 16 * 10 + 1]) == (0x15, 0x40)
    assert (wp[2048 + 16 * 8], wp[2048 + 16 * 8 + 1]) == (0x13, 0x40)
    assert (wp[2048 + 16 * 5], wp[2048 + 16 * 5 + 1]) == (0x12, 0x40)
    assert (wp[2048 + 16 * 1], wp[2048 + 16 * 1 + 1]) == (0x11, 0x40)
    assert wp[16 * 10] == 0x40
    # row 3 (up 0) block 2: qs = (3*8+2)*16 + j = 0xA0 + j; lane row 8,
    # k-group 1, byte 0: elements 8, 12 = low nibbles of 0xA8, 0xAC -> 0xC8
    assert wp[16 * (16 * 1 + 8) + 4 * 2 + 0] == 0xC8


@pytest.mark.parametrize("n,k,gated", [(40, 512, False), (37, 768, True), (16, 256, False)])
def test_repack_is_lossless(n, k, gated):
    """Every code and scale of every row reappears at its place: decoding the
    packed bytes back (loops over the layout's definition) gives the
    dequantised matrix, and the packed size is the GGUF size rounded up to
    whole row groups."""
    rows = 2 * n if gated else n
    blocks = oq.make_blocks(rows, k, seed=n + k)
    wp = oq.repack(blocks, n, k, gated)
    G, nc = oq.packed_groups(n, gated), k // 256
    assert wp.size == G * nc * 2304
    w = oq.dequant_f32(blocks, rows, k)
    got = np.full((rows, k), np.nan, dtype=np.float32)
    for Gi in range(G):
        for c in range(nc):
            ch = wp[(Gi * nc + c) * 2304:(Gi * nc + c + 1) * 2304]
            for r in range(16):
                if gated:
                    row = (n + min(8 * Gi + r - 8, n - 1)) if r >= 8 else min(8 * Gi + r, n - 1)
                else:
                    row = min(16 * Gi + r, n - 1)
                scales = ch[2048 + 16 * r:2048 + 16 * r + 16].copy().view("<f2").astype(np.float32)
                for g in range(4):
                    for blk in range(8):
                        off = (blk // 4) * 1024 + 16 * (16 * g + r) + 4 * (blk % 4)
                        for b in range(4):
                            byte = int(ch[off + b])
                            for e, code in ((8 * g + b, byte & 15), (8 * g + 4 + b, byte >> 4)):
                                got[row, c * 256 + blk * 32 + e] = scales[blk] * (code - 8)
    np.testing.assert_array_equal(got, w)
