"""Quantization plugin API (mirror of the reference's ``draco.quantization``)
with the GGUF backend registered, as ``draco/quantization/_register_all.py``
registers the reference's backends on import."""

from dracort_amd.quantization.base import QuantizationBackend  # noqa: F401
from dracort_amd.quantization.gguf import GGUFBackend, GGUFLinear, GGUFQuantizedWeight  # noqa: F401
from dracort_amd.quantization.quantize import (  # noqa: F401
    quantize,
    quantize_q4_0,
    quantize_q4_k,
    quantize_q6_k,
    quantize_q8_0,
)
from dracort_amd.quantization.registry import QUANT_REGISTRY, QuantizationRegistry  # noqa: F401

QUANT_REGISTRY.register("gguf", GGUFBackend())
