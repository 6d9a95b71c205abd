"""Plain-loop block decoders (oracle only).

K-quants restate the reference's independent test decoders ``_ref_q2_k``,
``_ref_q3_k``, ``_gsm``, ``_ref_q4_k``, ``_ref_q5_k``, ``_ref_q6_k`` and
``_ref_q8_k`` (``tests/format/test_gguf.py:232-341``), which follow the
element loops of ggml's ``dequantize_row_*`` rather than the vectorized
``_dequantize``.  Q4_1 / Q5_0 / Q5_1, which the reference tests only through
encoder round trips, follow the same published ggml loops (per block: element
j and j + 16 from byte j of qs; Q5's fifth bits from the 32-bit qh word).

One block at a time, element by element, in Python float64 with a final cast
to float32.  For these formats every product and difference of a float16
scale, a <= 6-bit scale and a <= 8-bit code is exact in float64, so the cast is
the only rounding and the loops agree bit-for-bit with a decoder that rounds
the exact value once; they pin element order, nibble/bit selection, scale
indexing and that single rounding.
"""

from __future__ import annotations

import numpy as np


def scale_min_k4(j: int, s12) -> tuple:
    """6-bit (scale, min) of sub-block j from the 12 packed scale bytes."""
    s = [int(v) for v in s12]
    if j < 4:
        return s[j] & 0x3F, s[j + 4] & 0x3F
    sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4)
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    return sc, m


def decode_q4_k_block(d: float, dmin: float, s12, qs) -> np.ndarray:
    vals = []
    for pair in range(4):
        lo_sc, lo_m = scale_min_k4(2 * pair, s12)
        hi_sc, hi_m = scale_min_k4(2 * pair + 1, s12)
        chunk = [int(v) for v in qs[32 * pair: 32 * pair + 32]]
        for byte in chunk:
            vals.append(d * lo_sc * (byte & 0x0F) - dmin * lo_m)
        for byte in chunk:
            vals.append(d * hi_sc * (byte >> 4) - dmin * hi_m)
    return np.asarray(vals, dtype=np.float32)


def decode_q6_k_block(d: float, ql, qh, sc) -> np.ndarray:
    """Returns the 256 values in natural element order."""
    out = [0.0] * 256
    ql = [int(v) for v in ql]
    qh = [int(v) for v in qh]
    sc = [int(v) for v in np.asarray(sc).astype(np.int8)]
    for half in range(2):
        for l in range(32):
            h = qh[32 * half + l]
            a = ql[64 * half + l]
            b = ql[64 * half + 32 + l]
            codes = (
                ((a & 0x0F) | ((h & 3) << 4)) - 32,
                ((b & 0x0F) | (((h >> 2) & 3) << 4)) - 32,
                ((a >> 4) | (((h >> 4) & 3) << 4)) - 32,
                ((b >> 4) | (((h >> 6) & 3) << 4)) - 32,
            )
            for t, q in enumerate(codes):
                s = sc[8 * half + l // 16 + 2 * t]
                out[128 * half + 32 * t + l] = d * s * q
    return np.asarray(out, dtype=np.float32)


def decode_q8_k_block(d: float, qs) -> np.ndarray:
    return np.asarray([d * int(v) for v in np.asarray(qs).astype(np.int8)], dtype=np.float32)


def decode_q2_k_block(d: float, dmin: float, qs, sc) -> np.ndarray:
    """qs[64], sc[16]: 16 runs of 16 elements, run r = (half, shift j, sub)."""
    qs = [int(v) for v in qs]
    sc = [int(v) for v in sc]
    vals = []
    run = 0
    for half in range(2):
        for j in range(4):
            for sub in range(2):
                s = sc[run]
                run += 1
                for l in range(16):
                    q = (qs[32 * half + 16 * sub + l] >> (2 * j)) & 3
                    vals.append(d * (s & 0x0F) * q - dmin * (s >> 4))
    return np.asarray(vals, dtype=np.float32)


def q3_k_scales(s12) -> list:
    """16 six-bit scales from 12 bytes, via the four 32-bit words ggml builds
    (low nibbles of words 0/1, high nibbles of words 0/1, each with two bits
    of word 2 on top)."""
    w = [int.from_bytes(bytes(np.asarray(s12, dtype=np.uint8)[4 * i: 4 * i + 4]), "little") for i in range(3)]
    lo4, hi2 = 0x0F0F0F0F, 0x03030303
    words = [(w[0] & lo4) | ((w[2] & hi2) << 4),
             (w[1] & lo4) | (((w[2] >> 2) & hi2) << 4),
             ((w[0] >> 4) & lo4) | (((w[2] >> 4) & hi2) << 4),
             ((w[1] >> 4) & lo4) | (((w[2] >> 6) & hi2) << 4)]
    return [(x >> (8 * b)) & 0xFF for x in words for b in range(4)]


def decode_q3_k_block(d: float, s12, qs, hm) -> np.ndarray:
    sc = q3_k_scales(s12)
    qs = [int(v) for v in qs]
    hm = [int(v) for v in hm]
    vals = []
    run = 0
    for half in range(2):
        for j in range(4):
            mask = 1 << (4 * half + j)
            for sub in range(2):
                dl = d * (sc[run] - 32)
                run += 1
                for l in range(16):
                    q = (qs[32 * half + 16 * sub + l] >> (2 * j)) & 3
                    vals.append(dl * (q - (0 if hm[16 * sub + l] & mask else 4)))
    return np.asarray(vals, dtype=np.float32)


def decode_q5_k_block(d: float, dmin: float, s12, qh, ql) -> np.ndarray:
    qh = [int(v) for v in qh]
    ql = [int(v) for v in ql]
    vals = []
    for pair in range(4):
        for nib in range(2):
            s = 2 * pair + nib
            sc, m = scale_min_k4(s, s12)
            for l in range(32):
                q = (ql[32 * pair + l] >> (4 * nib)) & 0x0F
                if (qh[l] >> s) & 1:
                    q += 16
                vals.append(d * sc * q - dmin * m)
    return np.asarray(vals, dtype=np.float32)


def decode_q4_1_block(d: float, m: float, qs) -> np.ndarray:
    out = [0.0] * 32
    for j, byte in enumerate(int(v) for v in qs):
        out[j] = (byte & 0x0F) * d + m
        out[j + 16] = (byte >> 4) * d + m
    return np.asarray(out, dtype=np.float32)


def decode_q5_block(d: float, m, qh_word: int, qs) -> np.ndarray:
    """Q5_0 (m is None: codes - 16) or Q5_1 (codes * d + m)."""
    out = [0.0] * 32
    for j, byte in enumerate(int(v) for v in qs):
        x0 = (byte & 0x0F) | (((qh_word >> j) << 4) & 0x10)
        x1 = (byte >> 4) | ((qh_word >> (j + 12)) & 0x10)
        if m is None:
            out[j], out[j + 16] = (x0 - 16) * d, (x1 - 16) * d
        else:
            out[j], out[j + 16] = x0 * d + m, x1 * d + m
    return np.asarray(out, dtype=np.float32)
