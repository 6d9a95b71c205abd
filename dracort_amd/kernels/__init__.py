"""GPU operators of the GGUF quantized-matmul path (HIP kernels, gfx950)."""

from dracort_amd.kernels.dense import dense_linear, get_rows, swiglu  # noqa: F401
from dracort_amd.kernels.glue import (  # noqa: F401
    DecodeAttentionWorkspace,
    decode_attention,
    decode_attention_workspace_bytes,
    rms_norm,
    rope_tables,
)
from dracort_amd.kernels.gguf import (  # noqa: F401
    block_layout,
    gemm_workspace_bytes,
    gguf_dequantize,
    gguf_gemm,
    gguf_gemv,
    gguf_gemv_multi,
    gguf_gemv_multi_rmsnorm,
    gguf_gemv_residual,
    gemv_residual_workspace_bytes,
    gguf_gemv_swiglu,
    gguf_gemv_swiglu_rmsnorm,
    gguf_linear,
    gguf_moe,
    moe_workspace_bytes,
)

__all__ = [
    "gguf_dequantize",
    "gguf_linear",
    "gguf_gemv",
    "gguf_gemv_multi",
    "gguf_gemv_swiglu",
    "gguf_gemv_multi_rmsnorm",
    "gguf_gemv_swiglu_rmsnorm",
    "gguf_gemv_residual",
    "gemv_residual_workspace_bytes",
    "gguf_gemm",
    "gguf_moe",
    "moe_workspace_bytes",
    "gemm_workspace_bytes",
    "block_layout",
    "rms_norm",
    "decode_attention",
    "decode_attention_workspace_bytes",
    "DecodeAttentionWorkspace",
    "rope_tables",
    "dense_linear",
    "get_rows",
    "swiglu",
]
