"""Pins the oracle's Q4_1 / Q5_0 / Q5_1 / Q8_K / Q2_K / Q3_K / Q5_K decoders
and the upstream field orders (no GPU needed).

* the reference's own known-answer K-quant blocks (tests/format/test_gguf.py:433-514
  of the reference: the same seeded draws, d / dmin / scale bytes) decoded by
  the restated plain-loop decoders;
* the loop decoders against the vectorized oracle on random blocks whose
  float16 fields cover normal, subnormal, zero, negative and extreme values:
  every intermediate of these formats is exact in float64, so the two must
  agree bit for bit;
* closed forms (unit scales give the raw codes in element order, exhaustive
  Q3_K 6-bit scale unpacking, code placement through the documented bit
  positions);
* the reference's encoder round-trip bounds for Q4_1 / Q5_0 / Q5_1
  (tests/format/test_gguf.py:412-430);
* planted mistakes (a shifted fifth bit, an inverted Q3_K high-bit mask,
  swapped Q2_K scale / min nibbles, Q3_K high scale bits from the wrong byte,
  an off-by-one Q5_K qh bit, a misread field order) must each be caught.
"""

import numpy as np
import pytest

from oracle import encoders, gguf_ref, loop_ref

Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K, Q8_K = 3, 6, 7, 10, 11, 13, 15
F16_SPECIAL = np.array([0x0000, 0x8000, 0x7BFF, 0xFBFF, 0x0400, 0x0001, 0x3C00, 0xBC00], dtype=np.uint16)


def _f16_pool(rng, n):
    """float16 bit patterns: normal, wide, subnormal and special values."""
    out = (rng.normal(size=n) * 0.05).astype(np.float16).view(np.uint16).copy()
    kind = rng.integers(0, 4, size=n)
    wide = (rng.normal(size=n) * 300.0).astype(np.float16).view(np.uint16)
    sub = rng.integers(1, 0x400, size=n, dtype=np.uint16) | (rng.integers(0, 2, size=n, dtype=np.uint16) << 15)
    out[kind == 1] = wide[kind == 1]
    out[kind == 2] = sub[kind == 2]
    out[kind == 3] = F16_SPECIAL[rng.integers(0, F16_SPECIAL.size, size=n)][kind == 3]
    return out


def _f16(bits) -> float:
    return float(np.uint16(bits).view(np.float16))


def _random_blocks(qtype, nb, seed):
    """Random block bytes with float16 fields drawn from the pool (reference order)."""
    rng = np.random.default_rng(seed)
    nbytes = gguf_ref.BLOCK_LAYOUT[qtype][1]
    b = rng.integers(0, 256, size=(nb, nbytes), dtype=np.uint8)
    f16_at = {Q4_1: [0, 2], Q5_0: [0], Q5_1: [0, 2], Q8_K: [0], Q2_K: [0, 2], Q3_K: [0], Q5_K: [0, 2]}[qtype]
    for off in f16_at:
        bits = _f16_pool(rng, nb)
        b[:, off] = (bits & 0xFF).astype(np.uint8)
        b[:, off + 1] = (bits >> 8).astype(np.uint8)
    return b


def _loop_decode(qtype, blk):
    """One block through the plain-loop decoders (reference field order)."""
    u16 = lambda o: _f16(int(blk[o]) | (int(blk[o + 1]) << 8))  # noqa: E731
    if qtype == Q4_1:
        return loop_ref.decode_q4_1_block(u16(0), u16(2), blk[4:20])
    if qtype in (Q5_0, Q5_1):
        o = 4 if qtype == Q5_1 else 2
        word = int.from_bytes(bytes(blk[o:o + 4]), "little")
        return loop_ref.decode_q5_block(u16(0), u16(2) if qtype == Q5_1 else None, word, blk[o + 4:o + 20])
    if qtype == Q8_K:
        return loop_ref.decode_q8_k_block(u16(0), blk[2:258].view(np.int8))
    if qtype == Q2_K:
        return loop_ref.decode_q2_k_block(u16(0), u16(2), blk[4:68], blk[68:84])
    if qtype == Q3_K:
        return loop_ref.decode_q3_k_block(u16(0), blk[2:14], blk[14:78], blk[78:110])
    return loop_ref.decode_q5_k_block(u16(0), u16(2), blk[4:16], blk[16:48], blk[48:176])


NEW_TYPES = [Q4_1, Q5_0, Q5_1, Q8_K, Q2_K, Q3_K, Q5_K]


def _expected(qtype, blocks):
    return np.concatenate([_loop_decode(qtype, blk) for blk in blocks])


# --- the reference's known-answer blocks --------------------------------------

def _reference_draws():
    """default_rng(11) draws in the order of the reference's K-quant test."""
    rng = np.random.default_rng(11)
    q2_qs = rng.integers(0, 256, 64, dtype=np.uint8)
    q3_qs = rng.integers(0, 256, 64, dtype=np.uint8)
    rng.integers(0, 256, 128, dtype=np.uint8)  # Q4_K qs
    q5_qh = rng.integers(0, 256, 32, dtype=np.uint8)
    q5_ql = rng.integers(0, 256, 128, dtype=np.uint8)
    rng.integers(0, 256, 128, dtype=np.uint8)  # Q6_K ql
    rng.integers(0, 256, 64, dtype=np.uint8)   # Q6_K qh
    q8_qs = rng.integers(-128, 128, 256, dtype=np.int8)
    return q2_qs, q3_qs, q5_qh, q5_ql, q8_qs


def test_reference_known_answer_blocks():
    q2_qs, q3_qs, q5_qh, q5_ql, q8_qs = _reference_draws()
    f16 = lambda v: np.float16(v).tobytes()  # noqa: E731
    # Q2_K: d = 1, dmin = 0.5, every scale byte 0x11
    sc = np.full(16, 0x11, np.uint8)
    got = gguf_ref.dequantize(Q2_K, f16(1.0) + f16(0.5) + q2_qs.tobytes() + sc.tobytes(), 256)
    assert np.array_equal(got, loop_ref.decode_q2_k_block(1.0, 0.5, q2_qs, sc))
    # Q3_K: d = 2, scale bytes 0x21, one hmask bit set
    s12 = np.full(12, 0x21, np.uint8)
    hm = np.zeros(32, np.uint8)
    hm[5] = 0x01
    got = gguf_ref.dequantize(Q3_K, f16(2.0) + s12.tobytes() + q3_qs.tobytes() + hm.tobytes(), 256)
    assert np.array_equal(got, loop_ref.decode_q3_k_block(2.0, s12, q3_qs, hm))
    # Q5_K: d = dmin = 1, scale bytes 0x01
    s12 = np.full(12, 0x01, np.uint8)
    got = gguf_ref.dequantize(Q5_K, f16(1.0) + f16(1.0) + s12.tobytes() + q5_qh.tobytes() + q5_ql.tobytes(), 256)
    assert np.array_equal(got, loop_ref.decode_q5_k_block(1.0, 1.0, s12, q5_qh, q5_ql))
    # Q8_K: d = 0.25
    got = gguf_ref.dequantize(Q8_K, f16(0.25) + q8_qs.tobytes(), 256)
    assert np.array_equal(got, loop_ref.decode_q8_k_block(0.25, q8_qs))


@pytest.mark.parametrize("qtype", NEW_TYPES)
def test_loop_decoders_agree_bitwise_on_random_blocks(qtype):
    qk = gguf_ref.BLOCK_LAYOUT[qtype][0]
    nb = 96 if qk == 32 else 24
    blocks = _random_blocks(qtype, nb, seed=100 + qtype)
    got = gguf_ref.dequantize(qtype, blocks, nb * qk)
    assert np.array_equal(got.view(np.uint32), _expected(qtype, blocks).view(np.uint32))


# --- closed forms ----------------------------------------------------------------

def test_q4_1_unit_scale_codes_and_offset():
    rng = np.random.default_rng(1)
    qs = rng.integers(0, 256, 16, dtype=np.uint8)
    codes = np.concatenate([qs & 15, qs >> 4]).astype(np.float32)
    blk = np.float16(1.0).tobytes() + np.float16(0.0).tobytes() + qs.tobytes()
    assert np.array_equal(gguf_ref.dequantize(Q4_1, blk, 32), codes)
    blk = np.float16(0.5).tobytes() + np.float16(-3.0).tobytes() + qs.tobytes()
    assert np.array_equal(gguf_ref.dequantize(Q4_1, blk, 32), codes * 0.5 - 3.0)


@pytest.mark.parametrize("qtype", [Q5_0, Q5_1])
def test_q5_code_placement(qtype):
    """Codes 0..31 placed through the documented bits: element e's low nibble in
    byte e % 16 (low nibble for e < 16), its fifth bit at bit e of qh."""
    codes = np.random.default_rng(2).permutation(32)
    qs = np.zeros(16, np.uint8)
    word = 0
    for e, c in enumerate(codes):
        qs[e % 16] |= (c & 15) << (4 * (e // 16))
        word |= (c >> 4) << e
    head = np.float16(1.0).tobytes() + (np.float16(0.0).tobytes() if qtype == Q5_1 else b"")
    blk = head + int(word).to_bytes(4, "little") + qs.tobytes()
    expect = codes.astype(np.float32) - (16 if qtype == Q5_0 else 0)
    assert np.array_equal(gguf_ref.dequantize(qtype, blk, 32), expect)


def test_q8_k_closed_form():
    codes = np.arange(-128, 128, dtype=np.int8)
    for d in (1.0, 0.0, -0.125):
        got = gguf_ref.dequantize(Q8_K, np.float16(d).tobytes() + codes.tobytes(), 256)
        assert np.array_equal(got, codes.astype(np.float32) * np.float32(d))


def _pack_q3k_scales(sc):
    """12 bytes from 16 six-bit scales, written from the bit layout."""
    b = [0] * 12
    for i, v in enumerate(sc):
        b[i % 8] |= (v & 15) << (4 * (i // 8))
        b[8 + i % 4] |= (v >> 4) << (2 * (i // 4))
    return np.array(b, dtype=np.uint8)


def test_q3k_scales_exhaustive():
    for v in range(64):
        for i in range(16):
            sc = [(63 - v + 5 * j) % 64 for j in range(16)]
            sc[i] = v
            s12 = _pack_q3k_scales(sc)
            assert list(gguf_ref.q3k_scales(s12)) == sc
            assert loop_ref.q3_k_scales(s12) == sc


def test_q3k_unit_scales_give_codes():
    """Scale 33 (33 - 32 = 1), d = 1: hmask bit set -> code, clear -> code - 4."""
    rng = np.random.default_rng(3)
    qs = rng.integers(0, 256, 64, dtype=np.uint8)
    hm = rng.integers(0, 256, 32, dtype=np.uint8)
    s12 = _pack_q3k_scales([33] * 16)
    got = gguf_ref.dequantize(Q3_K, np.float16(1.0).tobytes() + s12.tobytes() + qs.tobytes() + hm.tobytes(), 256)
    for e in range(256):
        half, r = divmod(e, 128)
        j, r = divmod(r, 32)
        sub, l = divmod(r, 16)
        low = (int(qs[32 * half + 16 * sub + l]) >> (2 * j)) & 3
        high = (int(hm[16 * sub + l]) >> (4 * half + j)) & 1
        assert got[e] == low + 4 * high - 4


def test_q2k_unit_scales_give_codes():
    rng = np.random.default_rng(4)
    qs = rng.integers(0, 256, 64, dtype=np.uint8)
    sc = np.full(16, 0x01, np.uint8)  # scale 1, min 0
    got = gguf_ref.dequantize(Q2_K, np.float16(1.0).tobytes() + np.float16(7.0).tobytes() + qs.tobytes()
                              + sc.tobytes(), 256)
    for e in range(256):
        half, r = divmod(e, 128)
        j, r = divmod(r, 32)
        sub, l = divmod(r, 16)
        assert got[e] == (int(qs[32 * half + 16 * sub + l]) >> (2 * j)) & 3
    # the min nibble: scale 0, min 1 -> every element is -dmin
    sc = np.full(16, 0x10, np.uint8)
    got = gguf_ref.dequantize(Q2_K, np.float16(1.0).tobytes() + np.float16(7.0).tobytes() + qs.tobytes()
                              + sc.tobytes(), 256)
    assert np.array_equal(got, np.full(256, -7.0, np.float32))


def test_q5k_fifth_bits():
    """Unit scales: element l of sub-block s is its nibble + 16 * bit s of qh[l]."""
    rng = np.random.default_rng(5)
    qh = rng.integers(0, 256, 32, dtype=np.uint8)
    ql = rng.integers(0, 256, 128, dtype=np.uint8)
    s12 = np.zeros(12, np.uint8)
    s12[0:4] = 1
    s12[8:12] = 1  # scales 1 for sub-blocks 0..7, mins 0
    got = gguf_ref.dequantize(Q5_K, np.float16(1.0).tobytes() + np.float16(0.0).tobytes() + s12.tobytes()
                              + qh.tobytes() + ql.tobytes(), 256).reshape(8, 32)
    for s in range(8):
        nib = (ql.reshape(4, 32)[s // 2] >> (4 * (s % 2))) & 15
        assert np.array_equal(got[s], (nib + 16 * ((qh >> s) & 1)).astype(np.float32))


# --- upstream field order -----------------------------------------------------------

@pytest.mark.parametrize("qtype", [Q2_K, Q3_K, 14])
def test_ggml_order_is_a_pure_field_move(qtype):
    qk = 256
    blocks = _random_blocks(qtype, 12, seed=7) if qtype != 14 else \
        np.random.default_rng(7).integers(0, 256, (12, 210), dtype=np.uint8)
    with np.errstate(invalid="ignore"):  # random Q6_K d bytes include NaN / Inf
        ref = gguf_ref.dequantize(qtype, blocks, 12 * qk)
        up = gguf_ref.to_ggml_order(qtype, blocks)
        assert not np.array_equal(up, blocks.reshape(-1))
        got = gguf_ref.dequantize(qtype, up, 12 * qk, ggml_order=True)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(gguf_ref.from_ggml_order(qtype, up), blocks.reshape(-1))


def test_ggml_order_field_positions():
    """ggml's structs: block_q2_K = scales[16] | qs[64] | d | dmin,
    block_q3_K = hmask[32] | qs[64] | scales[12] | d."""
    b = np.zeros((1, 84), np.uint8)
    b[0, 80:82] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    b[0, 0:16] = 0x01                 # scale 1, min 0
    b[0, 16:80] = 0xFF                # every 2-bit code = 3
    assert np.array_equal(gguf_ref.dequantize(Q2_K, b, 256, ggml_order=True), np.full(256, 6.0, np.float32))
    b = np.zeros((1, 110), np.uint8)
    b[0, 0:32] = 0xFF                 # every high bit set
    b[0, 32:96] = 0xAA                # every 2-bit code = 2
    b[0, 96:108] = _pack_q3k_scales([34] * 16)  # 34 - 32 = 2
    b[0, 108:110] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    assert np.array_equal(gguf_ref.dequantize(Q3_K, b, 256, ggml_order=True), np.full(256, 2.0, np.float32))


def test_single_order_types_reject_ggml_order():
    with pytest.raises(ValueError):
        gguf_ref.dequantize(Q5_K, bytes(176), 256, ggml_order=True)


# --- encoders -------------------------------------------------------------------------

def test_encoder_round_trip_tolerances():
    """The reference's own round-trip bounds (tests/format/test_gguf.py:412-430)."""
    x = (np.random.default_rng(3).normal(size=64) * 2.0).astype(np.float32)
    for qtype, enc, tol in ((Q4_1, encoders.enc_q4_1, 0.6), (Q5_0, encoders.enc_q5_0, 0.6),
                            (Q5_1, encoders.enc_q5_1, 0.4)):
        assert np.max(np.abs(gguf_ref.dequantize(qtype, enc(x), 64) - x)) < tol


def test_affine_encoders_exact_on_grid_values():
    """Values on the encoder's own grid (min + d * code, all exact) come back exactly."""
    rng = np.random.default_rng(8)
    for qtype, enc, top in ((Q4_1, encoders.enc_q4_1, 15), (Q5_1, encoders.enc_q5_1, 31)):
        codes = rng.integers(0, top + 1, (4, 32))
        codes[:, 0], codes[:, 1] = 0, top
        x = (-2.0 + 0.25 * codes).astype(np.float32)
        assert np.array_equal(gguf_ref.dequantize(qtype, enc(x.reshape(-1)), x.size).reshape(4, 32), x)


# --- planted mistakes ------------------------------------------------------------------

def _mut_q5_fifth_bit_unshifted(b):
    """Fifth bit of elements 16..31 taken from bit j + 12 without the shift."""
    b = b.copy()
    word = b[:, 2:6].copy().view(np.uint32)[:, 0]
    hi = (word >> np.uint32(16)) & np.uint32(0xFFFF)
    lo = word & np.uint32(0xFFFF)
    moved = lo | (((hi >> np.uint32(4)) & np.uint32(0x0FFF)) << np.uint32(16))
    b[:, 2:6] = moved.astype(np.uint32).view(np.uint8).reshape(-1, 4)
    return gguf_ref.dequantize(Q5_0, b, b.shape[0] * 32)


def _mut_q3k_mask_inverted(b):
    b = b.copy()
    b[:, 78:110] ^= 0xFF
    return gguf_ref.dequantize(Q3_K, b, b.shape[0] * 256)


def _mut_q2k_scale_min_swapped(b):
    b = b.copy()
    sc = b[:, 68:84]
    b[:, 68:84] = (sc >> 4) | (sc << 4)
    return gguf_ref.dequantize(Q2_K, b, b.shape[0] * 256)


def _mut_q3k_high_bits_wrong_byte(b):
    b = b.copy()
    b[:, 10:14] = b[:, 10:14][:, [1, 0, 3, 2]]
    return gguf_ref.dequantize(Q3_K, b, b.shape[0] * 256)


def _mut_q5k_qh_bit_off_by_one(b):
    b = b.copy()
    qh = b[:, 16:48]
    b[:, 16:48] = (qh << 1) | (qh >> 7)
    return gguf_ref.dequantize(Q5_K, b, b.shape[0] * 256)


def _mut_q2k_order_misread(b):
    return gguf_ref.dequantize(Q2_K, b, b.shape[0] * 256, ggml_order=True)


@pytest.mark.parametrize("qtype,mutant", [
    (Q5_0, _mut_q5_fifth_bit_unshifted), (Q3_K, _mut_q3k_mask_inverted), (Q2_K, _mut_q2k_scale_min_swapped),
    (Q3_K, _mut_q3k_high_bits_wrong_byte), (Q5_K, _mut_q5k_qh_bit_off_by_one), (Q2_K, _mut_q2k_order_misread)])
def test_planted_mistakes_are_caught(qtype, mutant):
    blocks = _random_blocks(qtype, 16, seed=200 + qtype)
    with np.errstate(all="ignore"):
        got = mutant(blocks)
    assert not np.array_equal(got.view(np.uint32), _expected(qtype, blocks).view(np.uint32))
