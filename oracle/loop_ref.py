"""Plain-loop K-quant decoders (oracle only).

Restates the reference's independent test decoders ``_gsm``, ``_ref_q4_k``
and ``_ref_q6_k`` (``tests/format/test_gguf.py:281-337``): one block at a time,
element by element, in Python arithmetic (float64) with a final cast to
float32.  Like the reference's, they agree bit-for-bit with the vectorized
decoder only where every intermediate is exact (small-integer scales, as in the
reference's known-answer blocks, ``tests/format/test_gguf.py:466-507``); they
pin element order, nibble/bit selection and scale indexing, not rounding.
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
