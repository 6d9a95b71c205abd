"""Registry of quantization backends, same interface as the reference's
``QuantizationRegistry`` / ``QUANT_REGISTRY`` (``draco/quantization/registry.py:21-90``)."""

from __future__ import annotations

import logging
from typing import Any, Dict, List, Optional

from dracort_amd.quantization.base import QuantizationBackend

logger = logging.getLogger("dracort_amd.quantization.registry")


class QuantizationRegistry:
    def __init__(self) -> None:
        self._backends: Dict[str, QuantizationBackend] = {}

    def register(self, name: str, backend: QuantizationBackend) -> None:
        key = name.lower()
        if key in self._backends:
            logger.warning(
                "Re-registering quantization backend '%s': %s -> %s",
                key, type(self._backends[key]).__name__, type(backend).__name__,
            )
        self._backends[key] = backend

    def get(self, name: str) -> QuantizationBackend:
        key = name.lower()
        if key not in self._backends:
            raise ValueError(f"Unknown quantization method: {key!r}. Available: {self.list_methods()}")
        return self._backends[key]

    def has(self, name: str) -> bool:
        return name.lower() in self._backends

    def list_methods(self) -> List[str]:
        return sorted(self._backends)

    def list_backends(self) -> Dict[str, QuantizationBackend]:
        return dict(self._backends)

    def detect_from_config(self, quantization_config: Dict[str, Any]) -> Optional[str]:
        method = quantization_config.get("quant_method", quantization_config.get("quantization_method"))
        if method and method.lower() in self._backends:
            return method.lower()
        return None

    def __contains__(self, name: str) -> bool:
        return self.has(name)

    def __len__(self) -> int:
        return len(self._backends)

    def __repr__(self) -> str:
        return f"QuantizationRegistry(methods={self.list_methods()})"


QUANT_REGISTRY = QuantizationRegistry()
