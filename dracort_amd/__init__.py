"""dracort_amd -- MI355X (gfx950) GGUF quantized-matmul path of DracoRT.

GGUF block dequantization (Q8_0, Q4_0, Q4_K, Q6_K) fused into the decode GEMV,
the prefill GEMM and the MoE expert matmuls, as hand-written HIP kernels in
``libdraco_gguf.so`` (C ABI: ``include/draco_gguf.h``) driven from Python
through ctypes with PyTorch-ROCm tensors as buffers.

Operator API (mirrors the reference's ``draco.kernels`` namespace and
``draco.quantization`` plugin registry):

    from dracort_amd.kernels import gguf_dequantize, gguf_linear, gguf_moe
    from dracort_amd.quantization import QUANT_REGISTRY
    QUANT_REGISTRY.get("gguf").quantized_linear(x, weight)
"""

from dracort_amd.exceptions import DracoError, DracoFormatError, KernelError, QuantizationError

__all__ = ["DracoError", "DracoFormatError", "KernelError", "QuantizationError"]
__version__ = "0.1.0"
