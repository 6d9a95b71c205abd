"""Quantization backend interface.

Same abstract interface as the reference's ``QuantizationBackend``
(``draco/quantization/base.py:17-133``) so a GGUF backend registered here is
called exactly like the reference's GPTQ/AWQ/FP8 backends.  One deliberate
difference: the reference's default ``quantized_linear`` passes ``weight`` in
place of ``scales`` to ``dequantize`` (``draco/quantization/base.py:98``); this
default passes ``scales``.
"""

from __future__ import annotations

import abc
from typing import Any, Dict, List, Optional

import torch
import torch.nn as nn


class QuantizationBackend(abc.ABC):
    @property
    @abc.abstractmethod
    def name(self) -> str: ...

    @property
    @abc.abstractmethod
    def supported_bits(self) -> List[int]: ...

    @property
    @abc.abstractmethod
    def supported_schemes(self) -> List[str]: ...

    @abc.abstractmethod
    def load_quantized_weights(
        self, model_path: str, target_model: nn.Module, config: Dict[str, Any], device: torch.device
    ) -> nn.Module: ...

    @abc.abstractmethod
    def dequantize(
        self,
        weights: torch.Tensor,
        scales: torch.Tensor,
        zeros: Optional[torch.Tensor] = None,
        group_size: int = 128,
    ) -> torch.Tensor: ...

    def quantized_linear(
        self,
        input: torch.Tensor,
        weight: torch.Tensor,
        scales: torch.Tensor,
        zeros: Optional[torch.Tensor] = None,
        bias: Optional[torch.Tensor] = None,
    ) -> torch.Tensor:
        """input @ dequantize(weight).T + bias"""
        return torch.nn.functional.linear(input, self.dequantize(weight, scales, zeros), bias)

    def supports_gpu_kernel(self, device: torch.device) -> bool:
        return device.type == "cuda"

    def get_kernel_info(self) -> Dict[str, Any]:
        return {"backend": self.name, "gpu_kernel": False, "optimized": False}

    def estimate_memory(self, num_params: int, bits: int, group_size: int = 128) -> int:
        quantized_bytes = num_params * bits // 8
        num_groups = num_params // group_size
        return quantized_bytes + num_groups * 2 + (num_groups * 2 if group_size > 0 else 0)

    def __repr__(self) -> str:
        return f"{self.__class__.__name__}(name={self.name!r}, bits={self.supported_bits})"
