"""GGUF block formats handled by the GPU path."""

from dracort_amd.format.gguf import (  # noqa: F401
    BLOCK_LAYOUTS,
    GGML_ORDER,
    GGML_TYPE_Q2_K,
    GGML_TYPE_Q3_K,
    GGML_TYPE_Q4_0,
    GGML_TYPE_Q4_1,
    GGML_TYPE_Q4_K,
    GGML_TYPE_Q5_0,
    GGML_TYPE_Q5_1,
    GGML_TYPE_Q5_K,
    GGML_TYPE_Q6_K,
    GGML_TYPE_Q8_0,
    GGML_TYPE_Q8_K,
    ORDER_TYPES,
    Q6K_D_LAST,
    GgufTensorInfo,
    layout,
    row_bytes,
    tensor_bytes,
)
