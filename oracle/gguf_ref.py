"""numpy restatement of the reference GGUF block dequantizer (oracle only).

Follows ``draco/format/gguf.py`` of the reference:

* block geometry ``_BLOCK_LAYOUTS`` / ``GGML_TYPE_*``   -> gguf.py:55-87
* ``_f16_from_u8``                                      -> gguf.py:256-259
* ``_dequantize`` type/size checks                      -> gguf.py:272-298
* Q8_0 branch                                           -> gguf.py:300-303
* Q8_K branch                                           -> gguf.py:305-308
* Q4_0 branch                                           -> gguf.py:310-316
* Q4_1 branch                                           -> gguf.py:318-324
* Q5_0 / Q5_1 branch                                    -> gguf.py:326-353
* Q2_K branch                                           -> gguf.py:355-374
* Q3_K branch                                           -> gguf.py:376-423
* Q4_K / Q5_K branch incl. ``_scale_min``               -> gguf.py:425-468
* Q6_K branch                                           -> gguf.py:470-495

The arithmetic keeps the reference's numpy dtypes so the fp32 rounding
sequence is the reference's:

* Q8_0 / Q8_K / Q4_0 / Q5_0: ``fl32(q * d)``           (exact: no rounding)
* Q4_1 / Q5_1: ``fl32(fl32(q * d) + m)``                (product exact: one rounding)
* Q4_K:        ``fl32(fl32(fl32(d*sc) * q) - fl32(dmin*m))``  (one rounding)
* Q2_K / Q5_K: ``fl32(d*sc)`` times an int32 code array is promoted to float64
               by numpy, the float32 ``fl32(dmin*m)`` is subtracted in float64;
               both steps are exact (the operands span < 53 bits), and the
               value is rounded once to float32 -- where Q5_K stores into a
               float32 array and where Q2_K's float64 result is cast by the
               kernel's ``matmul_f32`` (draco/runtime/cpu/kernels/generic.py:32-33).
* Q3_K:        ``fl32(d*(sc-32))`` times a code in -4..3: exact.
* Q6_K:        ``dl = fl32(d*sc)``; ``dl * q`` promoted to float64 by numpy
               (float32 array times int32 array), which is exact, then stored
               into a float32 array: one rounding, i.e. ``fl32(dl*q)``.

Field order.  The reference reads Q2_K, Q3_K and Q6_K blocks with their
float16 scale(s) first (d, dmin, qs, scales / d, scales, qs, hmask / d, ql,
qh, scales); the upstream ggml structs put them last (scales, qs, d, dmin /
hmask, qs, scales, d / ql, qh, scales, d).  ``ggml_order=True`` decodes the
upstream order; ``to_ggml_order`` / ``from_ggml_order`` move the fields (pure
byte moves).  Every other type has one order.
"""

from __future__ import annotations

from typing import Dict, Tuple

import numpy as np

GGML_TYPE_Q4_0 = 2
GGML_TYPE_Q4_1 = 3
GGML_TYPE_Q5_0 = 6
GGML_TYPE_Q5_1 = 7
GGML_TYPE_Q8_0 = 8
GGML_TYPE_Q2_K = 10
GGML_TYPE_Q3_K = 11
GGML_TYPE_Q4_K = 12
GGML_TYPE_Q5_K = 13
GGML_TYPE_Q6_K = 14
GGML_TYPE_Q8_K = 15

# (elements per block, bytes per block) -- gguf.py:75-87
BLOCK_LAYOUT: Dict[int, Tuple[int, int]] = {
    GGML_TYPE_Q4_0: (32, 18),
    GGML_TYPE_Q4_1: (32, 20),
    GGML_TYPE_Q5_0: (32, 22),
    GGML_TYPE_Q5_1: (32, 24),
    GGML_TYPE_Q8_0: (32, 34),
    GGML_TYPE_Q8_K: (256, 258),
    GGML_TYPE_Q2_K: (256, 84),
    GGML_TYPE_Q3_K: (256, 110),
    GGML_TYPE_Q4_K: (256, 144),
    GGML_TYPE_Q5_K: (256, 176),
    GGML_TYPE_Q6_K: (256, 210),
}

TYPE_NAMES = {
    GGML_TYPE_Q4_0: "Q4_0", GGML_TYPE_Q4_1: "Q4_1", GGML_TYPE_Q5_0: "Q5_0", GGML_TYPE_Q5_1: "Q5_1",
    GGML_TYPE_Q8_0: "Q8_0", GGML_TYPE_Q8_K: "Q8_K", GGML_TYPE_Q2_K: "Q2_K", GGML_TYPE_Q3_K: "Q3_K",
    GGML_TYPE_Q4_K: "Q4_K", GGML_TYPE_Q5_K: "Q5_K", GGML_TYPE_Q6_K: "Q6_K",
}

# Field spans (start, end) in the reference order and in the upstream ggml
# order, for the types whose two orders differ.
FIELD_SPANS = {
    GGML_TYPE_Q2_K: ({"d": (0, 4), "qs": (4, 68), "sc": (68, 84)},
                     {"sc": (0, 16), "qs": (16, 80), "d": (80, 84)}),
    GGML_TYPE_Q3_K: ({"d": (0, 2), "sc": (2, 14), "qs": (14, 78), "hm": (78, 110)},
                     {"hm": (0, 32), "qs": (32, 96), "sc": (96, 108), "d": (108, 110)}),
    GGML_TYPE_Q6_K: ({"d": (0, 2), "ql": (2, 130), "qh": (130, 194), "sc": (194, 210)},
                     {"ql": (0, 128), "qh": (128, 192), "sc": (192, 208), "d": (208, 210)}),
}


def f16_from_u8(pair: np.ndarray) -> np.ndarray:
    """(..., 2) little-endian uint8 -> float32 via float16 (gguf.py:256-259)."""
    bits = pair[..., 0].astype(np.uint32) | (pair[..., 1].astype(np.uint32) << 8)
    return bits.astype(np.uint16).view(np.float16).astype(np.float32)


def _as_blocks(qtype: int, payload, n: int) -> np.ndarray:
    if qtype not in BLOCK_LAYOUT:
        raise ValueError(f"ggml type {qtype} is not handled by the oracle")
    qk, nbytes = BLOCK_LAYOUT[qtype]
    if n % qk != 0:
        raise ValueError(f"element count {n} is not a multiple of block size {qk}")
    nb = n // qk
    raw = np.frombuffer(bytes(payload), dtype=np.uint8) if not isinstance(payload, np.ndarray) \
        else np.ascontiguousarray(payload, dtype=np.uint8).reshape(-1)
    if raw.size != nb * nbytes:
        raise ValueError(f"payload has {raw.size} bytes, expected {nb * nbytes}")
    return raw.reshape(nb, nbytes)


def _fields(qtype: int, b: np.ndarray, ggml_order: bool) -> Dict[str, np.ndarray]:
    spans = FIELD_SPANS[qtype][1 if ggml_order else 0]
    return {name: b[:, lo:hi] for name, (lo, hi) in spans.items()}


def _nibble_codes(packed: np.ndarray) -> np.ndarray:
    """16 packed bytes per block -> 32 codes: low nibbles are elements 0..15,
    high nibbles elements 16..31 (gguf.py:312-315, 321-323)."""
    return np.concatenate([packed & 0x0F, packed >> 4], axis=1)


def _dq_q8_0(b: np.ndarray) -> np.ndarray:
    # gguf.py:300-303
    d = f16_from_u8(b[:, 0:2])
    q = b[:, 2:34].view(np.int8).astype(np.float32)
    return (q * d[:, None]).reshape(-1)


def _dq_q8_k(b: np.ndarray) -> np.ndarray:
    # gguf.py:305-308: float16 d, 256 int8 codes
    d = f16_from_u8(b[:, 0:2])
    q = b[:, 2:258].view(np.int8).astype(np.float32)
    return (q * d[:, None]).reshape(-1)


def _dq_q4_0(b: np.ndarray) -> np.ndarray:
    # gguf.py:310-316: split halves, low nibbles first
    d = f16_from_u8(b[:, 0:2])
    codes = _nibble_codes(b[:, 2:18]).astype(np.int32) - 8
    return (codes.astype(np.float32) * d[:, None]).reshape(-1)


def _dq_q4_1(b: np.ndarray) -> np.ndarray:
    # gguf.py:318-324: fl32(fl32(q * d) + m)
    d = f16_from_u8(b[:, 0:2])
    m = f16_from_u8(b[:, 2:4])
    q = _nibble_codes(b[:, 4:20]).astype(np.float32)
    return (q * d[:, None] + m[:, None]).reshape(-1)


def q5_fifth_bits(qh4: np.ndarray) -> np.ndarray:
    """(nb, 4) little-endian bytes -> (nb, 32) fifth code bit of each element:
    bit e of the 32-bit word belongs to element e (gguf.py:336-344)."""
    word = np.zeros(qh4.shape[0], dtype=np.uint32)
    for i in range(4):
        word |= qh4[:, i].astype(np.uint32) << np.uint32(8 * i)
    return ((word[:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & 1).astype(np.uint8)


def _dq_q5(b: np.ndarray, with_min: bool) -> np.ndarray:
    # gguf.py:326-353: Q5_0 = d | qh[4] | qs[16], Q5_1 = d | m | qh[4] | qs[16]
    d = f16_from_u8(b[:, 0:2])
    o = 4 if with_min else 2
    codes = _nibble_codes(b[:, o + 4:o + 20]) | (q5_fifth_bits(b[:, o:o + 4]) << 4)
    if not with_min:
        return ((codes.astype(np.int32) - 16).astype(np.float32) * d[:, None]).reshape(-1)
    m = f16_from_u8(b[:, 2:4])
    return (codes.astype(np.float32) * d[:, None] + m[:, None]).reshape(-1)


def _dq_q2_k(b: np.ndarray, ggml_order: bool = False) -> np.ndarray:
    # gguf.py:355-374.  Element (half, j, sub, l) = 128*half + 32*j + 16*sub + l
    # is bits 2j..2j+1 of qs[32*half + 16*sub + l]; its scale byte is
    # sc[8*half + 2*j + sub] (low nibble: scale, high nibble: min).
    nb = b.shape[0]
    f = _fields(GGML_TYPE_Q2_K, b, ggml_order)
    d = f16_from_u8(f["d"][:, 0:2])
    dmin = f16_from_u8(f["d"][:, 2:4])
    qs = f["qs"].reshape(nb, 2, 1, 2, 16)                             # half, -, sub, l
    shifts = (2 * np.arange(4, dtype=np.uint8)).reshape(1, 1, 4, 1, 1)
    codes = ((qs >> shifts) & 3).astype(np.int32)                      # half, j, sub, l
    sc = f["sc"].reshape(nb, 2, 4, 2)                                  # half, j, sub
    dl = d[:, None, None, None] * (sc & 0x0F).astype(np.float32)       # fl32(d * scale)
    ml = dmin[:, None, None, None] * (sc >> 4).astype(np.float32)      # fl32(dmin * min)
    val = dl[..., None] * codes - ml[..., None]                        # float64, exact
    return val.astype(np.float32).reshape(-1)


def q3k_scales(s12: np.ndarray) -> np.ndarray:
    """12 packed bytes -> 16 six-bit scales (0..63): scale i takes nibble i // 8
    of byte i % 8 as its low four bits and bits 2*(i // 4) .. +1 of byte
    8 + i % 4 as its top two (gguf.py:377-398)."""
    i = np.arange(16)
    low = (s12[..., i % 8] >> (4 * (i // 8)).astype(np.uint8)) & 0x0F
    high = (s12[..., 8 + i % 4] >> (2 * (i // 4)).astype(np.uint8)) & 3
    return low | (high << 4)


def _dq_q3_k(b: np.ndarray, ggml_order: bool = False) -> np.ndarray:
    # gguf.py:376-423.  Element (half, j, sub, l) has low bits 2j..2j+1 of
    # qs[32*half + 16*sub + l], high bit 4*half + j of hmask[16*sub + l]
    # (clear: subtract 4), scale sc[8*half + 2*j + sub] - 32.
    nb = b.shape[0]
    f = _fields(GGML_TYPE_Q3_K, b, ggml_order)
    d = f16_from_u8(f["d"])
    qs = f["qs"].reshape(nb, 2, 1, 2, 16)                              # half, -, sub, l
    hm = f["hm"].reshape(nb, 1, 1, 2, 16)                              # -, -, sub, l
    j = np.arange(4, dtype=np.uint8)
    low2 = ((qs >> (2 * j).reshape(1, 1, 4, 1, 1)) & 3).astype(np.int32)
    bit = (4 * np.arange(2, dtype=np.uint8)[:, None] + j[None, :]).reshape(1, 2, 4, 1, 1)
    high = ((hm >> bit) & 1).astype(np.int32)
    q = low2 - 4 * (1 - high)                                          # half, j, sub, l
    sc = q3k_scales(f["sc"]).astype(np.int32) - 32
    dl = (d[:, None] * sc.astype(np.float32)).reshape(nb, 2, 4, 2)     # fl32(d * (sc - 32))
    return (dl[..., None] * q).astype(np.float32).reshape(-1)          # exact product


def q4k_scale_min(sc12: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """12 packed bytes -> (scale[8], min[8]) 6-bit values (gguf.py:436-442)."""
    sc = np.empty(sc12.shape[:-1] + (8,), dtype=np.uint8)
    mn = np.empty_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j] = sc12[..., j] & 63
            mn[..., j] = sc12[..., j + 4] & 63
        else:
            sc[..., j] = (sc12[..., j + 4] & 0x0F) | ((sc12[..., j - 4] >> 6) << 4)
            mn[..., j] = (sc12[..., j + 4] >> 4) | ((sc12[..., j] >> 6) << 4)
    return sc, mn


def _dq_q4_k(b: np.ndarray) -> np.ndarray:
    # gguf.py:425-468 (Q4_K path)
    nb = b.shape[0]
    d = f16_from_u8(b[:, 0:2])
    dmin = f16_from_u8(b[:, 2:4])
    sc, mn = q4k_scale_min(b[:, 4:16])
    d_sub = d[:, None] * sc.astype(np.float32)       # fl32(d*sc), (nb, 8)
    m_sub = dmin[:, None] * mn.astype(np.float32)    # fl32(dmin*m), (nb, 8)
    qs = b[:, 16:144].reshape(nb, 4, 32)
    # sub-block 2g uses the low nibbles of qs[32g:32g+32], 2g+1 the high ones
    codes = np.stack([qs & 0x0F, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.float32)
    prod = d_sub[:, :, None] * codes                 # fl32(d1*q)
    out = prod - m_sub[:, :, None]                   # fl32(. - m1)
    return out.reshape(-1)


def _dq_q5_k(b: np.ndarray) -> np.ndarray:
    # gguf.py:425-468 (Q5_K path): bit s of qh[l] is the fifth bit of element
    # l of sub-block s; value fl32(d*sc) * code - fl32(dmin*m) in float64
    # (exact), stored as float32.
    nb = b.shape[0]
    d = f16_from_u8(b[:, 0:2])
    dmin = f16_from_u8(b[:, 2:4])
    sc, mn = q4k_scale_min(b[:, 4:16])
    d_sub = d[:, None] * sc.astype(np.float32)
    m_sub = dmin[:, None] * mn.astype(np.float32)
    qh = b[:, 16:48]
    qs = b[:, 48:176].reshape(nb, 4, 32)
    low4 = np.stack([qs & 0x0F, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.int32)
    fifth = ((qh[:, None, :] >> np.arange(8, dtype=np.uint8)[None, :, None]) & 1).astype(np.int32)
    val = d_sub[:, :, None] * (low4 + 16 * fifth) - m_sub[:, :, None]
    return val.astype(np.float32).reshape(-1)


def _dq_q6_k(b: np.ndarray, ggml_order: bool = False) -> np.ndarray:
    # gguf.py:470-495
    nb = b.shape[0]
    f = _fields(GGML_TYPE_Q6_K, b, ggml_order)
    ql, qh, sc8 = f["ql"], f["qh"], f["sc"]
    d = f16_from_u8(f["d"])
    sc = sc8.view(np.int8).astype(np.int32).reshape(nb, 2, 8)
    ql2 = ql.reshape(nb, 2, 64)
    qh2 = qh.reshape(nb, 2, 32)
    low4 = np.stack(
        [ql2[:, :, 0:32] & 0x0F, ql2[:, :, 32:64] & 0x0F, ql2[:, :, 0:32] >> 4, ql2[:, :, 32:64] >> 4],
        axis=2,
    )                                                # (nb, half, t, l)
    shifts = np.array([0, 2, 4, 6], dtype=np.uint8)[None, None, :, None]
    high2 = (qh2[:, :, None, :] >> shifts) & 3
    q = (low4 | (high2 << 4)).astype(np.int32) - 32  # (nb, half, t, l)
    # scale index within the half: l // 16 + 2 t
    t_idx = np.arange(4)[:, None]
    l_idx = np.arange(32)[None, :]
    sel = (l_idx // 16) + 2 * t_idx                  # (t, l)
    dl = d[:, None, None, None] * sc[:, :, sel].astype(np.float32)   # fl32(d*sc)
    out = (dl * q).astype(np.float32)                # f64 product (exact) -> one rounding
    return out.reshape(-1)


def dequantize(qtype: int, payload, n: int, ggml_order: bool = False) -> np.ndarray:
    """Flat float32 dequantization of ``n`` elements, as ``_dequantize`` (gguf.py:272).

    ``ggml_order``: Q2_K / Q3_K / Q6_K blocks in the upstream field order."""
    if ggml_order and qtype not in FIELD_SPANS:
        raise ValueError(f"ggml type {qtype} has a single field order")
    b = _as_blocks(qtype, payload, n)
    if qtype == GGML_TYPE_Q8_0:
        return _dq_q8_0(b)
    if qtype == GGML_TYPE_Q8_K:
        return _dq_q8_k(b)
    if qtype == GGML_TYPE_Q4_0:
        return _dq_q4_0(b)
    if qtype == GGML_TYPE_Q4_1:
        return _dq_q4_1(b)
    if qtype in (GGML_TYPE_Q5_0, GGML_TYPE_Q5_1):
        return _dq_q5(b, qtype == GGML_TYPE_Q5_1)
    if qtype == GGML_TYPE_Q2_K:
        return _dq_q2_k(b, ggml_order)
    if qtype == GGML_TYPE_Q3_K:
        return _dq_q3_k(b, ggml_order)
    if qtype == GGML_TYPE_Q4_K:
        return _dq_q4_k(b)
    if qtype == GGML_TYPE_Q5_K:
        return _dq_q5_k(b)
    return _dq_q6_k(b, ggml_order)


def dequantize_matrix(qtype: int, payload, shape, ggml_order: bool = False) -> np.ndarray:
    """[N, K] weight: numpy shape = reversed GGUF dims, blocks run along K (gguf.py:646-648)."""
    n_rows, k = int(shape[0]), int(shape[1])
    return dequantize(qtype, payload, n_rows * k, ggml_order).reshape(n_rows, k)


def _block_rows(qtype: int, payload) -> np.ndarray:
    nbytes = BLOCK_LAYOUT[qtype][1]
    raw = np.frombuffer(bytes(payload), dtype=np.uint8) if not isinstance(payload, np.ndarray) \
        else np.ascontiguousarray(payload, dtype=np.uint8).reshape(-1)
    return raw.reshape(-1, nbytes)


def _move_fields(qtype: int, payload, to_ggml: bool) -> np.ndarray:
    src, dst = FIELD_SPANS[qtype] if to_ggml else FIELD_SPANS[qtype][::-1]
    b = _block_rows(qtype, payload)
    out = np.empty_like(b)
    for name, (lo, hi) in src.items():
        dlo, dhi = dst[name]
        out[:, dlo:dhi] = b[:, lo:hi]
    return out.reshape(-1)


def to_ggml_order(qtype: int, payload) -> np.ndarray:
    """Reference field order -> upstream ggml order (pure byte move)."""
    return _move_fields(qtype, payload, True)


def from_ggml_order(qtype: int, payload) -> np.ndarray:
    """Upstream ggml field order -> reference order (pure byte move)."""
    return _move_fields(qtype, payload, False)


def q6k_reorder(payload, to_upstream: bool) -> np.ndarray:
    """Permute Q6_K fields between the reference order (d, ql, qh, sc) and the
    upstream ggml order (ql, qh, sc, d)."""
    return _move_fields(GGML_TYPE_Q6_K, payload, to_upstream)


def row_bytes(qtype: int, k: int) -> int:
    qk, nbytes = BLOCK_LAYOUT[qtype]
    return (k // qk) * nbytes
