"""GGUF quantization backend for the reference's plugin registry.

``GGUFBackend`` implements the reference's ``QuantizationBackend`` interface
(``draco/quantization/base.py:17-133``) for GGUF block weights and is
registered as ``QUANT_REGISTRY.register("gguf", GGUFBackend())`` the same way
the reference registers its backends (``draco/quantization/_register_all.py``).
A GGUF weight carries its scales inside its blocks, so the backend's weight
argument is a :class:`GGUFQuantizedWeight` (packed bytes in HBM + ggml type +
[N, K] shape) and ``scales`` / ``zeros`` are unused.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple, Union

import numpy as np
import torch
import torch.nn as nn

from dracort_amd.exceptions import QuantizationError
from dracort_amd.format.gguf import BITS_PER_WEIGHT, TYPE_NAMES, base_type, layout, tensor_bytes
from dracort_amd.kernels.gguf import gguf_dequantize, gguf_linear
from dracort_amd.quantization.base import QuantizationBackend


@dataclass
class GGUFQuantizedWeight:
    """Packed GGUF blocks of an [N, K] weight resident in device memory."""

    data: torch.Tensor          # uint8, N * (K / QK) * block_bytes
    ggml_type: int
    shape: Tuple[int, int]

    def __post_init__(self) -> None:
        layout(self.ggml_type)
        self.shape = (int(self.shape[0]), int(self.shape[1]))
        need = tensor_bytes(self.ggml_type, self.shape)
        if self.data.dtype != torch.uint8 or self.data.numel() != need:
            raise QuantizationError(
                f"GGUF {TYPE_NAMES.get(base_type(self.ggml_type), self.ggml_type)} weight {self.shape} needs "
                f"{need} uint8 bytes, got {self.data.numel()} {self.data.dtype}"
            )

    @classmethod
    def from_bytes(
        cls, payload: Union[bytes, np.ndarray, torch.Tensor], ggml_type: int, shape, device="cuda"
    ) -> "GGUFQuantizedWeight":
        if isinstance(payload, torch.Tensor):
            t = payload.reshape(-1).to(torch.uint8)
        else:
            t = torch.from_numpy(np.frombuffer(bytes(payload), dtype=np.uint8).copy())
        return cls(t.to(device), int(ggml_type), tuple(shape))

    @property
    def nbytes(self) -> int:
        return self.data.numel()

    @property
    def device(self) -> torch.device:
        return self.data.device

    def dequantize(self) -> torch.Tensor:
        return gguf_dequantize(self.data, self.ggml_type, self.shape)


class GGUFLinear(nn.Module):
    """``nn.Linear`` replacement holding a GGUF weight: y = x @ W.T + b (float32 out)."""

    def __init__(self, weight: GGUFQuantizedWeight, bias: Optional[torch.Tensor] = None) -> None:
        super().__init__()
        self.weight_q = weight
        self.register_buffer("qdata", weight.data, persistent=False)
        self.bias = None if bias is None else nn.Parameter(bias.to(torch.float32), requires_grad=False)
        self.out_features, self.in_features = weight.shape

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return gguf_linear(x.contiguous(), self.qdata, self.weight_q.ggml_type, self.weight_q.shape, self.bias)


class GGUFBackend(QuantizationBackend):
    @property
    def name(self) -> str:
        return "gguf"

    @property
    def supported_bits(self) -> List[int]:
        return [4, 6, 8]

    @property
    def supported_schemes(self) -> List[str]:
        return ["weight_only"]

    def load_quantized_weights(
        self, model_path: str, target_model: nn.Module, config: Dict[str, Any], device: torch.device
    ) -> nn.Module:
        """Swap ``nn.Linear`` submodules for :class:`GGUFLinear`.

        ``config["weights"]`` maps a submodule name to a
        :class:`GGUFQuantizedWeight` (or to ``(payload, ggml_type, shape)``);
        ``model_path`` is not read here (the weights are already decoded from
        their container).
        """
        weights = config.get("weights")
        if not weights:
            raise QuantizationError("GGUFBackend.load_quantized_weights needs config['weights']")
        modules = dict(target_model.named_modules())
        for name, spec in weights.items():
            if name not in modules:
                raise QuantizationError(f"no submodule named {name!r}")
            w = spec if isinstance(spec, GGUFQuantizedWeight) else GGUFQuantizedWeight.from_bytes(
                spec[0], spec[1], spec[2], device=device
            )
            old = modules[name]
            bias = getattr(old, "bias", None)
            new = GGUFLinear(w, None if bias is None else bias.detach().to(device))
            parent_name, _, child = name.rpartition(".")
            parent = modules[parent_name] if parent_name else target_model
            setattr(parent, child, new)
        return target_model

    def dequantize(
        self,
        weights: Union[GGUFQuantizedWeight, torch.Tensor],
        scales: Optional[torch.Tensor] = None,
        zeros: Optional[torch.Tensor] = None,
        group_size: int = 128,
        ggml_type: Optional[int] = None,
        shape: Optional[Tuple[int, int]] = None,
    ) -> torch.Tensor:
        w = self._as_weight(weights, ggml_type, shape)
        return gguf_dequantize(w.data, w.ggml_type, w.shape)

    def quantized_linear(
        self,
        input: torch.Tensor,
        weight: Union[GGUFQuantizedWeight, torch.Tensor],
        scales: Optional[torch.Tensor] = None,
        zeros: Optional[torch.Tensor] = None,
        bias: Optional[torch.Tensor] = None,
        ggml_type: Optional[int] = None,
        shape: Optional[Tuple[int, int]] = None,
    ) -> torch.Tensor:
        w = self._as_weight(weight, ggml_type, shape)
        b = None if bias is None else bias.to(torch.float32).contiguous()
        return gguf_linear(input.contiguous(), w.data, w.ggml_type, w.shape, b)

    def get_kernel_info(self) -> Dict[str, Any]:
        return {
            "backend": self.name,
            "gpu_kernel": True,
            "optimized": True,
            "arch": "gfx950",
            "types": sorted(TYPE_NAMES.values()),
            "kernels": ["dequant_f32", "gemv (M<=16)", "gemm (bf16 MFMA)", "moe_ffn"],
        }

    def estimate_memory(self, num_params: int, bits: int, group_size: int = 128) -> int:
        """Bytes of GGUF blocks for ``num_params`` weights at the nearest supported type."""
        per = {4: BITS_PER_WEIGHT[12], 6: BITS_PER_WEIGHT[14], 8: BITS_PER_WEIGHT[8]}.get(bits)
        if per is None:
            return super().estimate_memory(num_params, bits, group_size)
        return int(round(num_params * per / 8.0))

    @staticmethod
    def _as_weight(weight, ggml_type, shape) -> GGUFQuantizedWeight:
        if isinstance(weight, GGUFQuantizedWeight):
            return weight
        if ggml_type is None or shape is None:
            raise QuantizationError("a raw uint8 GGUF tensor needs ggml_type= and shape=")
        return GGUFQuantizedWeight(weight.reshape(-1), int(ggml_type), tuple(shape))
