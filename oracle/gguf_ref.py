"""numpy restatement of the reference GGUF block dequantizer (oracle only).

Follows ``draco/format/gguf.py`` of the reference:

* block geometry ``_BLOCK_LAYOUTS`` / ``GGML_TYPE_*``   -> gguf.py:55-87
* ``_f16_from_u8``                                      -> gguf.py:256-259
* ``_dequantize`` type/size checks                      -> gguf.py:272-298
* Q8_0 branch                                           -> gguf.py:300-303
* Q4_0 branch                                           -> gguf.py:310-316
* Q4_K branch incl. ``_scale_min``                      -> gguf.py:425-468
* Q6_K branch                                           -> gguf.py:470-495

The arithmetic is kept operation-for-operation in the same numpy dtypes so the
fp32 rounding sequence is the reference's:

* Q8_0 / Q4_0: ``fl32(q * d)``                        (one rounding)
* Q4_K:        ``fl32(fl32(fl32(d*sc) * q) - fl32(dmin*m))``
* Q6_K:        ``dl = fl32(d*sc)``; ``dl * q`` promoted to float64 by numpy
               (float32 array times int32 array), which is exact, then stored
               into a float32 array: one rounding, i.e. ``fl32(dl*q)``.

The Q6_K block is read in the reference's field order (d at bytes 0-1, then
ql[128], qh[64], scales[16]); ``q6k_reorder`` converts from/to the upstream
ggml order (ql, qh, scales, d) for layout-flag tests.
"""

from __future__ import annotations

from typing import Dict, Tuple

import numpy as np

GGML_TYPE_Q4_0 = 2
GGML_TYPE_Q8_0 = 8
GGML_TYPE_Q4_K = 12
GGML_TYPE_Q6_K = 14

# (elements per block, bytes per block) -- gguf.py:75-87
BLOCK_LAYOUT: Dict[int, Tuple[int, int]] = {
    GGML_TYPE_Q4_0: (32, 18),
    GGML_TYPE_Q8_0: (32, 34),
    GGML_TYPE_Q4_K: (256, 144),
    GGML_TYPE_Q6_K: (256, 210),
}

TYPE_NAMES = {
    GGML_TYPE_Q4_0: "Q4_0",
    GGML_TYPE_Q8_0: "Q8_0",
    GGML_TYPE_Q4_K: "Q4_K",
    GGML_TYPE_Q6_K: "Q6_K",
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


def _dq_q8_0(b: np.ndarray) -> np.ndarray:
    # gguf.py:300-303
    d = f16_from_u8(b[:, 0:2])
    q = b[:, 2:34].view(np.int8).astype(np.float32)
    return (q * d[:, None]).reshape(-1)


def _dq_q4_0(b: np.ndarray) -> np.ndarray:
    # gguf.py:310-316: split halves, low nibbles first
    d = f16_from_u8(b[:, 0:2])
    packed = b[:, 2:18]
    low = (packed & 0x0F).astype(np.int32) - 8
    high = (packed >> 4).astype(np.int32) - 8
    codes = np.concatenate([low, high], axis=1).astype(np.float32)
    return (codes * d[:, None]).reshape(-1)


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


def _q6k_fields(b: np.ndarray, d_last: bool):
    if d_last:
        return b[:, 0:128], b[:, 128:192], b[:, 192:208], b[:, 208:210]
    return b[:, 2:130], b[:, 130:194], b[:, 194:210], b[:, 0:2]


def _dq_q6_k(b: np.ndarray, d_last: bool = False) -> np.ndarray:
    # gguf.py:470-495
    nb = b.shape[0]
    ql, qh, sc8, dpair = _q6k_fields(b, d_last)
    d = f16_from_u8(dpair)
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


def dequantize(qtype: int, payload, n: int, q6k_d_last: bool = False) -> np.ndarray:
    """Flat float32 dequantization of ``n`` elements, as ``_dequantize`` (gguf.py:272)."""
    b = _as_blocks(qtype, payload, n)
    if qtype == GGML_TYPE_Q8_0:
        return _dq_q8_0(b)
    if qtype == GGML_TYPE_Q4_0:
        return _dq_q4_0(b)
    if qtype == GGML_TYPE_Q4_K:
        return _dq_q4_k(b)
    return _dq_q6_k(b, q6k_d_last)


def dequantize_matrix(qtype: int, payload, shape, q6k_d_last: bool = False) -> np.ndarray:
    """[N, K] weight: numpy shape = reversed GGUF dims, blocks run along K (gguf.py:646-648)."""
    n_rows, k = int(shape[0]), int(shape[1])
    return dequantize(qtype, payload, n_rows * k, q6k_d_last).reshape(n_rows, k)


def q6k_reorder(payload, to_upstream: bool) -> np.ndarray:
    """Permute Q6_K fields between the reference order (d, ql, qh, sc) and the
    upstream ggml order (ql, qh, sc, d).  Pure byte move, no arithmetic."""
    b = np.frombuffer(bytes(payload), dtype=np.uint8).reshape(-1, 210) if not isinstance(payload, np.ndarray) \
        else np.ascontiguousarray(payload, dtype=np.uint8).reshape(-1, 210)
    out = np.empty_like(b)
    if to_upstream:
        out[:, 0:208] = b[:, 2:210]
        out[:, 208:210] = b[:, 0:2]
    else:
        out[:, 2:210] = b[:, 0:208]
        out[:, 0:2] = b[:, 208:210]
    return out.reshape(-1)


def row_bytes(qtype: int, k: int) -> int:
    qk, nbytes = BLOCK_LAYOUT[qtype]
    return (k // qk) * nbytes
