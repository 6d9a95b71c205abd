"""GGUF block-format constants and shape rules for the quantized-matmul path.

Mirrors the reference's ggml type ids and ``_BLOCK_LAYOUTS``
(``draco/format/gguf.py:55-87``) for the eleven block types its
``_dequantize`` reads (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_K, Q2_K, Q3_K, Q4_K,
Q5_K, Q6_K), and its tensor shape rule: numpy/torch shape = GGUF dims
reversed, so an ``[N, K]`` weight has its blocks running along the contiguous
K axis (``draco/format/gguf.py:630-648``).

Field order.  The reference decodes Q2_K, Q3_K and Q6_K blocks with their
float16 scales first; upstream ggml files store them last.  ``GGML_ORDER``
(0x100) or'ed into a type id selects the upstream order for those three types
(``Q6K_D_LAST`` is its older name).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Tuple

from dracort_amd.exceptions import DracoFormatError

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

# Layout flag: Q2_K / Q3_K / Q6_K blocks in upstream ggml field order.
GGML_ORDER = 0x100
Q6K_D_LAST = GGML_ORDER
ORDER_TYPES = (GGML_TYPE_Q2_K, GGML_TYPE_Q3_K, GGML_TYPE_Q6_K)

# (elements per block, bytes per block)
BLOCK_LAYOUTS: Dict[int, Tuple[int, int]] = {
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
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}

# effective bits per weight of each type
BITS_PER_WEIGHT = {t: 8.0 * nb / qk for t, (qk, nb) in BLOCK_LAYOUTS.items()}


def base_type(ggml_type: int) -> int:
    return int(ggml_type) & ~GGML_ORDER


def layout(ggml_type: int) -> Tuple[int, int]:
    base = base_type(ggml_type)
    if base not in BLOCK_LAYOUTS:
        raise DracoFormatError(
            f"GGUF quantization type {ggml_type} is not supported by this build "
            f"(supported: Q4_0=2, Q4_1=3, Q5_0=6, Q5_1=7, Q8_0=8, Q2_K=10, Q3_K=11, Q4_K=12, Q5_K=13, "
            f"Q6_K=14, Q8_K=15)."
        )
    if base != int(ggml_type) and base not in ORDER_TYPES:
        raise DracoFormatError(f"layout flag GGML_ORDER applies to Q2_K, Q3_K and Q6_K only (got {ggml_type}).")
    return BLOCK_LAYOUTS[base]


def row_bytes(ggml_type: int, k: int) -> int:
    qk, nb = layout(ggml_type)
    if k % qk != 0:
        raise DracoFormatError(
            f"GGUF row length {k} is not divisible by block size {qk} for ggml type {ggml_type}."
        )
    return (k // qk) * nb


def tensor_bytes(ggml_type: int, shape: Tuple[int, int]) -> int:
    n, k = int(shape[0]), int(shape[1])
    return n * row_bytes(ggml_type, k)


@dataclass
class GgufTensorInfo:
    """Duck-typed counterpart of the reference's ``GgufTensorInfo``
    (``draco/format/gguf.py:504-520``) for a 2-D quantized weight."""

    name: str
    ggml_type: int
    shape: Tuple[int, ...]
    offset: int = 0
    nbytes: int = 0
    alignment: int = 32
    dtype: str = "f32"
    quantization: Optional[str] = None
