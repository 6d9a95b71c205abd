"""Pins the CPU oracle before it is trusted as the checker (no GPU needed).

* golden vectors written by running the reference ``_dequantize`` and test
  encoders (tests/golden/make_golden.py);
* the reference's own known-answer K-quant blocks and plain-loop decoders
  (tests/format/test_gguf.py:433-514 of the reference);
* closed forms fixed by the arithmetic (unit scales, zero scales, exact
  products, exhaustive 6-bit scale/min unpacking, element order);
* planted mistakes: each plausible slip (dropped high scale bits, swapped
  nibbles, a wrong Q6_K scale index, the wrong Q6_K field order, a reordered
  Q6_K product) applied to the oracle must be caught by these fixtures.

Note on rounding: for Q8_0, Q4_0 and Q4_K every product of a float16 scale
(11-bit significand) with 6-bit scales and <= 8-bit codes is exact in float32,
so the only rounding is Q4_K's final subtraction; an FMA there gives the same
bits.  Q6_K's product fl(d*sc) * q has up to 25 significant bits and does
round, so its evaluation order matters and is pinned.
"""

import os

import numpy as np
import pytest

from oracle import encoders, gguf_ref, loop_ref, matmul_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = [("Q4_0", 2), ("Q8_0", 8), ("Q4_K", 12), ("Q6_K", 14)]


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "gguf_dequant_golden.npz"))


@pytest.fixture(scope="module")
def enc_golden():
    return np.load(os.path.join(GOLDEN, "gguf_encoder_golden.npz"))


@pytest.mark.parametrize("name,qtype", TYPES)
def test_oracle_matches_reference_golden(golden, name, qtype):
    blocks = golden[f"{name}_blocks"]
    qk = gguf_ref.BLOCK_LAYOUT[qtype][0]
    got = gguf_ref.dequantize(qtype, blocks, blocks.shape[0] * qk)
    assert np.array_equal(got.view(np.uint32), golden[f"{name}_expect_bits"])


def test_q6k_upstream_order_is_a_pure_field_move(golden):
    blocks = golden["Q6_K_blocks"]
    up = gguf_ref.q6k_reorder(blocks, to_upstream=True)
    assert not np.array_equal(up, blocks.reshape(-1))
    got = gguf_ref.dequantize(14, up, blocks.shape[0] * 256, ggml_order=True)
    assert np.array_equal(got.view(np.uint32), golden["Q6_K_expect_bits"])
    assert np.array_equal(gguf_ref.q6k_reorder(up, to_upstream=False), blocks.reshape(-1))


def _reference_known_answer_blocks():
    """The reference test's draws from default_rng(11), in its order
    (tests/format/test_gguf.py:433-514): Q2_K qs, Q3_K qs, Q4_K qs, Q5_K qh/ql, Q6_K ql/qh."""
    rng = np.random.default_rng(11)
    rng.integers(0, 256, 64, dtype=np.uint8)   # Q2_K qs
    rng.integers(0, 256, 64, dtype=np.uint8)   # Q3_K qs
    q4k_qs = rng.integers(0, 256, 128, dtype=np.uint8)
    rng.integers(0, 256, 32, dtype=np.uint8)   # Q5_K qh
    rng.integers(0, 256, 128, dtype=np.uint8)  # Q5_K ql
    q6k_ql = rng.integers(0, 256, 128, dtype=np.uint8)
    q6k_qh = rng.integers(0, 256, 64, dtype=np.uint8)
    return q4k_qs, q6k_ql, q6k_qh


def test_reference_known_answer_blocks():
    q4k_qs, q6k_ql, q6k_qh = _reference_known_answer_blocks()
    # Q4_K: d = dmin = 1.0, all scale bytes 0x01
    s12 = np.full(12, 0x01, dtype=np.uint8)
    payload = np.float16(1.0).tobytes() + np.float16(1.0).tobytes() + s12.tobytes() + q4k_qs.tobytes()
    got = gguf_ref.dequantize(12, payload, 256)
    assert np.array_equal(got, loop_ref.decode_q4_k_block(1.0, 1.0, s12, q4k_qs))
    # Q6_K: d = 1.5, int8 scales all 2
    sc = np.full(16, 2, dtype=np.int8)
    payload = np.float16(1.5).tobytes() + q6k_ql.tobytes() + q6k_qh.tobytes() + sc.tobytes()
    got = gguf_ref.dequantize(14, payload, 256)
    assert np.array_equal(got, loop_ref.decode_q6_k_block(1.5, q6k_ql, q6k_qh, sc))


def test_loop_decoders_on_golden_blocks_with_small_integer_scales(golden):
    """With power-of-two d/dmin every intermediate is exact, so the loop decoders
    (float64) and the vectorized float32 decoder must agree bit-for-bit."""
    rng = np.random.default_rng(17)
    for _ in range(20):
        s12 = rng.integers(0, 256, 12, dtype=np.uint8)
        qs = rng.integers(0, 256, 128, dtype=np.uint8)
        d, dmin = 2.0 ** rng.integers(-8, 3), 2.0 ** rng.integers(-8, 3)
        payload = np.float16(d).tobytes() + np.float16(dmin).tobytes() + s12.tobytes() + qs.tobytes()
        assert np.array_equal(gguf_ref.dequantize(12, payload, 256), loop_ref.decode_q4_k_block(d, dmin, s12, qs))
        ql = rng.integers(0, 256, 128, dtype=np.uint8)
        qh = rng.integers(0, 256, 64, dtype=np.uint8)
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        payload = np.float16(d).tobytes() + ql.tobytes() + qh.tobytes() + sc.tobytes()
        assert np.array_equal(gguf_ref.dequantize(14, payload, 256), loop_ref.decode_q6_k_block(d, ql, qh, sc))


def test_q8_0_closed_forms():
    codes = np.arange(-128, 128, dtype=np.int8).reshape(-1, 32)
    for d, expect in ((1.0, codes.astype(np.float32)), (0.0, np.zeros(codes.shape, np.float32)),
                      (0.125, codes.astype(np.float32) / 8)):
        blocks = np.concatenate(
            [np.tile(np.frombuffer(np.float16(d).tobytes(), np.uint8), (codes.shape[0], 1)), codes.view(np.uint8)], 1
        )
        got = gguf_ref.dequantize(8, blocks, codes.size).reshape(codes.shape)
        assert np.array_equal(got, expect)
    # arbitrary d: the product of an int8 and a float16 is exact in float64, so the
    # float32 result must be its single correctly-rounded value
    rng = np.random.default_rng(2)
    dvals = (rng.normal(size=64) * 3).astype(np.float16)
    blocks = np.zeros((64, 34), np.uint8)
    blocks[:, 0:2] = dvals.view(np.uint8).reshape(64, 2)
    blocks[:, 2:] = rng.integers(0, 256, (64, 32), dtype=np.uint8)
    got = gguf_ref.dequantize(8, blocks, 64 * 32).reshape(64, 32)
    exact = blocks[:, 2:].view(np.int8).astype(np.float64) * dvals.astype(np.float64)[:, None]
    assert np.array_equal(got, exact.astype(np.float32))


def test_q4_0_element_order_and_offset():
    lo = np.arange(16, dtype=np.uint8)          # elements 0..15 -> codes 0..15
    hi = (15 - np.arange(16)).astype(np.uint8)  # elements 16..31 -> codes 15..0
    block = np.concatenate([np.frombuffer(np.float16(1.0).tobytes(), np.uint8), lo | (hi << 4)])
    got = gguf_ref.dequantize(2, block, 32)
    assert np.array_equal(got, np.concatenate([lo, hi]).astype(np.float32) - 8)


def _pack_q4k_scales(sc, mn):
    """12 scale bytes from 6-bit (scale, min) pairs, written from the bit layout:
    j<4 -> low 6 bits of bytes j / j+4; j>=4 -> nibbles of byte j+4 plus the top
    2 bits of bytes j-4 (scale) and j (min)."""
    b = [0] * 12
    for j in range(8):
        if j < 4:
            b[j] |= sc[j] & 63
            b[j + 4] |= mn[j] & 63
        else:
            b[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
            b[j - 4] |= (sc[j] >> 4) << 6
            b[j] |= (mn[j] >> 4) << 6
    return np.array(b, dtype=np.uint8)


def test_q4k_scale_min_exhaustive():
    for v in range(64):
        for j in range(8):
            sc = [0] * 8
            mn = [63 - v] * 8
            sc[j] = v
            s12 = _pack_q4k_scales(sc, mn)
            got_sc, got_mn = gguf_ref.q4k_scale_min(s12[None, :])
            assert list(got_sc[0]) == sc and list(got_mn[0]) == mn


def test_q4k_unit_scales_give_raw_nibbles():
    rng = np.random.default_rng(4)
    qs = rng.integers(0, 256, 128, dtype=np.uint8)
    s12 = _pack_q4k_scales([1] * 8, [0] * 8)
    payload = np.float16(1.0).tobytes() + np.float16(0.0).tobytes() + s12.tobytes() + qs.tobytes()
    got = gguf_ref.dequantize(12, payload, 256).reshape(4, 2, 32)
    assert np.array_equal(got[:, 0, :], (qs.reshape(4, 32) & 15).astype(np.float32))
    assert np.array_equal(got[:, 1, :], (qs.reshape(4, 32) >> 4).astype(np.float32))


def test_q6k_code_order_round_trip():
    """Place known 6-bit codes at every element through the documented bit
    positions and read them back with unit scales."""
    rng = np.random.default_rng(9)
    codes = rng.integers(0, 64, 256)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e, q in enumerate(codes):
        half, r = divmod(e, 128)
        t, l = divmod(r, 32)
        byte = 64 * half + l + 32 * (t & 1)
        ql[byte] |= (q & 15) << (4 * (t >> 1))
        qh[32 * half + l] |= (q >> 4) << (2 * t)
    payload = np.float16(1.0).tobytes() + ql.tobytes() + qh.tobytes() + np.ones(16, np.int8).tobytes()
    assert np.array_equal(gguf_ref.dequantize(14, payload, 256), (codes - 32).astype(np.float32))


# --- planted mistakes: the fixtures above must catch each of them -------------

def _dq_q4k_scale_high_bits_dropped(b):
    """Sub-blocks 4..7 read only the low nibble of their scale / min."""
    nb = b.shape[0]
    d = gguf_ref.f16_from_u8(b[:, 0:2])
    dmin = gguf_ref.f16_from_u8(b[:, 2:4])
    sc, mn = gguf_ref.q4k_scale_min(b[:, 4:16])
    sc[:, 4:] &= 15
    mn[:, 4:] &= 15
    qs = b[:, 16:144].reshape(nb, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.float32)
    d1 = d[:, None] * sc.astype(np.float32)
    m1 = dmin[:, None] * mn.astype(np.float32)
    return (d1[:, :, None] * q - m1[:, :, None]).reshape(-1)


def _dq_q6k_product_order(b):
    """fl(fl(d*q)*sc) instead of fl(fl(d*sc)*q): the 25-bit product rounds differently."""
    ref = gguf_ref.dequantize(14, b, b.shape[0] * 256).reshape(-1, 256)
    d = gguf_ref.f16_from_u8(b[:, 0:2])
    sc_all = b[:, 194:210].view(np.int8).astype(np.float32)
    out = np.empty_like(ref)
    for e in range(256):
        half, r = divmod(e, 128)
        t, l = divmod(r, 32)
        s = sc_all[:, 8 * half + l // 16 + 2 * t]
        with np.errstate(invalid="ignore"):
            q = np.where(s != 0, ref[:, e] / np.where(s != 0, d * s, 1), 0).round()
        out[:, e] = (d * q.astype(np.float32)) * s
    return out.reshape(-1)


def _dq_q4k_swapped_nibbles(b):
    b = b.copy()
    qs = b[:, 16:144]
    b[:, 16:144] = (qs >> 4) | (qs << 4)
    return gguf_ref.dequantize(12, b, b.shape[0] * 256)


def _dq_q6k_wrong_scale_index(b):
    nb = b.shape[0]
    sc = b[:, 194:210].view(np.int8).reshape(nb, 2, 8)
    perm = b.copy()
    perm[:, 194:210] = sc[:, :, [0, 2, 1, 3, 4, 6, 5, 7]].reshape(nb, 16).view(np.uint8)
    return gguf_ref.dequantize(14, perm, nb * 256)


def _dq_q6k_d_last_misread(b):
    return gguf_ref.dequantize(14, b, b.shape[0] * 256, ggml_order=True)


@pytest.mark.parametrize(
    "name,mutant",
    [("Q4_K", _dq_q4k_scale_high_bits_dropped), ("Q4_K", _dq_q4k_swapped_nibbles),
     ("Q6_K", _dq_q6k_wrong_scale_index), ("Q6_K", _dq_q6k_d_last_misread), ("Q6_K", _dq_q6k_product_order)],
)
def test_planted_mistakes_are_caught(golden, name, mutant):
    got = mutant(golden[f"{name}_blocks"])
    assert not np.array_equal(got.view(np.uint32), golden[f"{name}_expect_bits"])


# --- encoders ------------------------------------------------------------------

@pytest.mark.parametrize("tag", ["small", "wide", "zero"])
def test_encoders_match_reference_golden(enc_golden, tag):
    x = enc_golden[f"x_{tag}"]
    assert np.array_equal(np.frombuffer(encoders.enc_q8_0(x), np.uint8), enc_golden[f"q8_0_{tag}"])
    assert np.array_equal(np.frombuffer(encoders.enc_q4_0(x), np.uint8), enc_golden[f"q4_0_{tag}"])


def test_encoder_round_trip_tolerances():
    """The reference's own round-trip bounds (tests/format/test_gguf.py:412-430)."""
    x = (np.random.default_rng(3).normal(size=64) * 2.0).astype(np.float32)
    assert np.max(np.abs(gguf_ref.dequantize(8, encoders.enc_q8_0(x), 64) - x)) < 0.05
    assert np.max(np.abs(gguf_ref.dequantize(2, encoders.enc_q4_0(x), 64) - x)) < 1.0


# --- matmul / MoE closed forms ---------------------------------------------------

def test_linear_ref_brute_force():
    rng = np.random.default_rng(5)
    x = rng.normal(size=(3, 7)).astype(np.float32)
    w = rng.normal(size=(5, 7)).astype(np.float32)
    ref = matmul_ref.linear_ref(x, w)
    for i in range(3):
        for j in range(5):
            assert abs(ref[i, j] - sum(float(x[i, k]) * float(w[j, k]) for k in range(7))) < 1e-12
    assert ref.shape == (3, 5)


def test_rel_err_metric():
    ref = np.array([1.0, -2.0, 1e-9, 4.0])
    assert matmul_ref.rel_err(ref, ref) == (0.0, 0.0)
    y = ref.copy()
    y[2] += 4e-3  # near-zero output: floor at 1e-3 * max|ref| = 4e-3 -> error 1.0
    elem, _ = matmul_ref.rel_err(y, ref)
    assert abs(elem - 1.0) < 1e-6
    y = ref * (1 + 5e-4)
    assert matmul_ref.rel_err(y, ref)[0] == pytest.approx(5e-4, rel=1e-6)


def test_route_ref_top2_softmax():
    logits = np.array([[0.1, 2.0, -1.0, 1.0], [3.0, 3.0, 0.0, -5.0]])
    idx, w = matmul_ref.route_ref(logits, 2)
    assert idx.tolist() == [[1, 3], [0, 1]]  # tie -> lower index first
    e = np.exp(1.0 - 2.0)
    assert w[0].tolist() == pytest.approx([1 / (1 + e), e / (1 + e)])
    assert w[1].tolist() == pytest.approx([0.5, 0.5])
    assert np.allclose(w.sum(axis=1), 1.0)


def test_moe_ref_brute_force():
    rng = np.random.default_rng(6)
    t_, h, i_, e_ = 5, 4, 6, 3
    x = rng.normal(size=(t_, h))
    logits = rng.normal(size=(t_, e_))
    experts = [(rng.normal(size=(i_, h)), rng.normal(size=(i_, h)), rng.normal(size=(h, i_))) for _ in range(e_)]
    got = matmul_ref.moe_ref(x, logits, experts, 2)
    for t in range(t_):
        order = sorted(range(e_), key=lambda e: -logits[t, e])[:2]
        z = np.exp([logits[t, e] - logits[t, order[0]] for e in order])
        wts = z / z.sum()
        acc = np.zeros(h)
        for e, wt in sorted(zip(order, wts)):
            g = experts[e][0] @ x[t]
            u = experts[e][1] @ x[t]
            acc += wt * (experts[e][2] @ (g / (1 + np.exp(-g)) * u))
        assert np.allclose(got[t], acc, rtol=1e-12, atol=1e-12)
