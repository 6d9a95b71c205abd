"""Reference Q8_0 / Q4_0 encoders (oracle only).

Restates the reference's test encoders ``_enc_q8_0`` and ``_enc_q4_0``
(``tests/format/test_gguf.py:145-169``), which are the only GGUF quantizers the
reference has and therefore the quantizer of the Q8_0 / Q4_0 configurations.
Quirks kept on purpose:

* the block scale is computed in float32 as ``max(amax, 1e-12) / 127`` (Q8_0)
  or ``/ 8`` (Q4_0); the codes are rounded with that float32 scale while the
  *stored* scale is its float16 rounding;
* ``rint`` is round-half-to-even;
* Q4_0 stores ``clip(rint(x/d) + 8, 0, 15)``, so ``+amax`` saturates at 15,
  low nibbles hold elements 0..15 and high nibbles 16..31.
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
