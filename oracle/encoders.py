"""Reference Q8_0 / Q4_0 / Q4_1 / Q5_0 / Q5_1 encoders (oracle only).

Restates the reference's test encoders ``_enc_q8_0``, ``_enc_q4_0``,
``_enc_q4_1``, ``_enc_q5_0`` and ``_enc_q5_1``
(``tests/format/test_gguf.py:145-229``), which are the only GGUF quantizers the
reference has and therefore the quantizer of the Q8_0 / Q4_0 configurations.
Quirks kept on purpose:

* the block scale is computed in float32 as ``max(amax, 1e-12) / 127`` (Q8_0)
  or ``/ 8`` (Q4_0); the codes are rounded with that float32 scale while the
  *stored* scale is its float16 rounding;
* ``rint`` is round-half-to-even;
* Q4_0 stores ``clip(rint(x/d) + 8, 0, 15)``, so ``+amax`` saturates at 15,
  low nibbles hold elements 0..15 and high nibbles 16..31;
* Q5_0: ``d = max(amax, 1e-12) / 16``, codes ``clip(rint(x/d) + 16, 0, 31)``;
* Q4_1 / Q5_1: ``d = (max - min) / 15`` (``/ 31``), or 1 when the span is
  <= 1e-12, offset ``min``; codes ``clip(rint((x - min)/d), 0, 15 | 31)``;
* Q5 fifth bits: bit e of the little-endian 32-bit qh word is bit 4 of the
  code of element e.
"""

from __future__ import annotations

import numpy as np


def enc_q8_0(values: np.ndarray) -> bytes:
    a = np.asarray(values, dtype=np.float32).reshape(-1, 32)
    nb = a.shape[0]
    scale = np.maximum(np.max(np.abs(a), axis=1), 1e-12) / 127.0
    codes = np.clip(np.rint(a / scale[:, None]), -127, 127).astype(np.int8)
    blocks = np.empty((nb, 34), dtype=np.uint8)
    blocks[:, 0:2] = scale.astype(np.float16).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:34] = codes.view(np.uint8)
    return blocks.tobytes()


def enc_q4_0(values: np.ndarray) -> bytes:
    a = np.asarray(values, dtype=np.float32).reshape(-1, 32)
    nb = a.shape[0]
    scale = np.maximum(np.max(np.abs(a), axis=1), 1e-12) / 8.0
    codes = np.clip(np.rint(a / scale[:, None]) + 8, 0, 15).astype(np.uint8)
    blocks = np.empty((nb, 18), dtype=np.uint8)
    blocks[:, 0:2] = scale.astype(np.float16).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:18] = codes[:, 0:16] | (codes[:, 16:32] << 4)
    return blocks.tobytes()


def _pack_nibbles(codes: np.ndarray) -> np.ndarray:
    return (codes[:, 0:16] & 0x0F) | ((codes[:, 16:32] & 0x0F) << 4)


def _fifth_bits(codes: np.ndarray) -> np.ndarray:
    word = np.zeros(codes.shape[0], dtype=np.uint32)
    for e in range(32):
        word |= ((codes[:, e] >> 4).astype(np.uint32) & 1) << np.uint32(e)
    return word.view(np.uint8).reshape(-1, 4)


def _affine_codes(a: np.ndarray, top: int):
    lo = np.min(a, axis=1)
    span = np.max(a, axis=1) - lo
    d = np.where(span > 1e-12, span / np.float32(top), np.float32(1.0)).astype(np.float32)
    codes = np.clip(np.rint((a - lo[:, None]) / d[:, None]), 0, top).astype(np.uint8)
    return d, lo, codes


def enc_q4_1(values: np.ndarray) -> bytes:
    a = np.asarray(values, dtype=np.float32).reshape(-1, 32)
    d, lo, codes = _affine_codes(a, 15)
    blocks = np.empty((a.shape[0], 20), dtype=np.uint8)
    blocks[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:4] = lo.astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 4:20] = _pack_nibbles(codes)
    return blocks.tobytes()


def enc_q5_0(values: np.ndarray) -> bytes:
    a = np.asarray(values, dtype=np.float32).reshape(-1, 32)
    d = np.maximum(np.max(np.abs(a), axis=1), 1e-12) / np.float32(16.0)
    codes = np.clip(np.rint(a / d[:, None]) + 16, 0, 31).astype(np.uint8)
    blocks = np.empty((a.shape[0], 22), dtype=np.uint8)
    blocks[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:6] = _fifth_bits(codes)
    blocks[:, 6:22] = _pack_nibbles(codes)
    return blocks.tobytes()


def enc_q5_1(values: np.ndarray) -> bytes:
    a = np.asarray(values, dtype=np.float32).reshape(-1, 32)
    d, lo, codes = _affine_codes(a, 31)
    blocks = np.empty((a.shape[0], 24), dtype=np.uint8)
    blocks[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:4] = lo.astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 4:8] = _fifth_bits(codes)
    blocks[:, 8:24] = _pack_nibbles(codes)
    return blocks.tobytes()
