"""GGUF block-format constants and shape rules for the quantized-matmul path.

Mirrors the reference's ggml type ids and ``_BLOCK_LAYOUTS``
(``draco/format/gguf.py:55-87``) for the four types this path runs on the
GPU, and its tensor shape rule: numpy/torch shape = GGUF dims reversed, so an
``[N, K]`` weight has its blocks running along the contiguous K axis
(``draco/format/gguf.py:630-648``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Tuple

from dracort_amd.exceptions import DracoFormatError

GGML_TYPE_Q4_0 = 2
GGML_TYPE_Q8_0 = 8
GGML_TYPE_Q4_K = 12
GGML_TYPE_Q6_K = 14

# Layout flag for Q6_K blocks stored in upstream ggml field order (d last).
Q6K_D_LAST = 0x100

# (elements per block, bytes per block)
BLOCK_LAYOUTS: Dict[int, Tuple[int, int]] = {
    GGML_TYPE_Q4_0: (32, 18),
    GGML_TYPE_Q8_0: (32, 34),
    GGML_TYPE_Q4_K: (256, 144),
    GGML_TYPE_Q6_K: (256, 210),
}

TYPE_NAMES = {GGML_TYPE_Q4_0: "Q4_0", GGML_TYPE_Q8_0: "Q8_0", GGML_TYPE_Q4_K: "Q4_K", GGML_TYPE_Q6_K: "Q6_K"}
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}

# effective bits per weight of each type
BITS_PER_WEIGHT = {t: 8.0 * nb / qk for t, (qk, nb) in BLOCK_LAYOUTS.items()}


def base_type(ggml_type: int) -> int:
    return int(ggml_type) & ~Q6K_D_LAST


def layout(ggml_type: int) -> Tuple[int, int]:
    base = base_type(ggml_type)
    if base not in BLOCK_LAYOUTS:
        raise DracoFormatError(
            f"GGUF quantization type {ggml_type} is not supported by this build "
            f"(supported: Q8_0=8, Q4_0=2, Q4_K=12, Q6_K=14)."
        )
    if base != int(ggml_type) and base != GGML_TYPE_Q6_K:
        raise DracoFormatError(f"layout flag Q6K_D_LAST applies to Q6_K only (got {ggml_type}).")
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
