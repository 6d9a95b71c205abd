"""GPU kernel tier for the executor's ``_linear`` on GGUF tensors.

The reference executor routes every projection through ``_linear``
(``draco/runtime/cpu/executor.py:47-79``): a GGUF tensor (its info carries
``quantization=None`` and a ``ggml_type``) is dequantized to float32 by
``reader.get_tensor`` and multiplied by the selected CPU kernel's
``matmul_f32``; the kernel objects follow ``CPUGemmKernel``
(``draco/runtime/cpu/kernels/base.py:10-31``: ``tier``, ``name``,
``supports(quantization)``, ``matmul(activation, tensor_info,
weight_bytes)``) and are held in a ``KernelSelection``
(``draco/runtime/cpu/dispatcher.py:30-35``).

:class:`GGUFGpuKernel` is that kind of object for the MI355X path.  It keeps
each GGUF weight's packed blocks resident in HBM after first use and runs
``gguf_linear`` on them.  A tier object may serve several readers (the
reference keeps its kernels as process-wide singletons,
``draco/runtime/cpu/dispatcher.py:25``), so the residency cache is keyed on
where the bytes come from, never on the tensor name alone: for ``linear`` the
file (real path, device, inode, size, modification time), the tensor name, its
offset and the kernel type (which carries the Q2_K / Q3_K / Q6_K field order);
for ``matmul`` the tensor name, kernel type, shape and a 128-bit hash of the
``weight_bytes`` handed in, so changed bytes are always uploaded again.

* ``matmul(activation, tensor_info, weight_bytes)`` -- the reference
  signature: numpy activations in, numpy float32 out (host <-> device copies
  around the fused kernel);
* ``linear(reader, name, x, bias_name=None)`` -- ``_linear`` itself for a
  GGUF tensor, with ``x`` a numpy array (returns numpy) or a device tensor
  (returns a device tensor, no host copies).

``reader`` is a :class:`~dracort_amd.format.gguf_file.GGUFFile` (payloads
read zero-copy from the mapping, Q6_K tagged with its field order) or the
reference's ``GGUFReader`` (``tensor_info``, ``_raw_bytes``, ``get_tensor``
for float biases).  There is no CPU fallback: without the HIP library or a
GPU every call raises.
"""

from __future__ import annotations

import hashlib
import os
from typing import Callable, Dict, Hashable, Optional, Tuple, Union

import numpy as np
import torch

from dracort_amd.exceptions import KernelError
from dracort_amd.format.gguf import BLOCK_LAYOUTS, base_type
from dracort_amd.format.gguf_file import GGUFFile
from dracort_amd.kernels.gguf import gguf_linear
from dracort_amd.quantization.gguf import GGUFQuantizedWeight

Array = Union[np.ndarray, torch.Tensor]

try:  # a fast 128-bit hash of the weight bytes (matmul's cache key); hashlib otherwise
    import xxhash

    def _digest(buf) -> bytes:
        return xxhash.xxh3_128_digest(buf)
except ImportError:  # pragma: no cover - xxhash ships with this image
    def _digest(buf) -> bytes:
        return hashlib.blake2b(buf, digest_size=16).digest()


def reader_key(reader) -> Hashable:
    """Identity of the file behind a reader: (real path, st_dev, st_ino, size,
    mtime_ns); a reader without a path is identified by the object itself."""
    path = getattr(reader, "path", None)
    if isinstance(path, (str, bytes, os.PathLike)):
        try:
            st = os.stat(path)
            return ("file", os.path.realpath(path), st.st_dev, st.st_ino, st.st_size, st.st_mtime_ns)
        except OSError:
            pass
    return ("reader", id(reader))


def linear_weight_key(reader, info, kernel_type: int) -> Hashable:
    return (reader_key(reader), info.name, int(info.offset), int(kernel_type))


def bytes_weight_key(info, kernel_type: int, weight_bytes) -> Hashable:
    buf = weight_bytes if isinstance(weight_bytes, (bytes, bytearray, memoryview)) else \
        np.ascontiguousarray(weight_bytes).view(np.uint8)
    return ("bytes", info.name, int(kernel_type), tuple(info.shape), _digest(buf))


def is_gguf_block_tensor(info) -> bool:
    """A 2-D GGUF tensor of a block type the kernels run."""
    return (getattr(info, "quantization", None) is None and getattr(info, "ggml_type", None) is not None
            and base_type(info.ggml_type) in BLOCK_LAYOUTS and len(info.shape) == 2)


class GGUFGpuKernel:
    """Executor kernel tier: fused dequant + GEMV / GEMM on HBM-resident GGUF blocks."""

    tier = "gpu-gguf"

    def __init__(self, device: Union[str, torch.device] = "cuda") -> None:
        self.device = torch.device(device)
        self._weights: Dict[Hashable, Union[GGUFQuantizedWeight, torch.Tensor]] = {}

    @property
    def name(self) -> str:
        return "mi355x-gguf"

    def supports(self, quantization: Optional[str]) -> bool:
        # GGUF tensor infos carry quantization=None; the block type decides (supports_tensor)
        return quantization is None

    def supports_tensor(self, info) -> bool:
        return is_gguf_block_tensor(info)

    # -- weights ---------------------------------------------------------
    def resident_weight(self, key: Hashable, info, kernel_type: int,
                        fetch: Callable[[], object]) -> GGUFQuantizedWeight:
        """The HBM copy of a tensor's packed blocks under cache key ``key``;
        ``fetch()`` gives the payload (bytes or a uint8 array) and is called
        on first use of the key only."""
        if not is_gguf_block_tensor(info):
            raise KernelError(f"tensor '{getattr(info, 'name', '?')}' is not a GGUF block tensor this tier runs")
        w = self._weights.get(key)
        if w is None:
            if not torch.cuda.is_available():
                raise KernelError("the GGUF GPU tier needs a GPU (no CPU fallback)")
            payload = np.frombuffer(fetch(), dtype=np.uint8)
            data = torch.from_numpy(payload.copy()).to(self.device)
            w = GGUFQuantizedWeight(data, int(kernel_type), tuple(info.shape))
            self._weights[key] = w
        return w

    def resident_bytes(self) -> int:
        return sum(w.nbytes if isinstance(w, GGUFQuantizedWeight) else w.numel() * w.element_size()
                   for w in self._weights.values())

    def evict(self) -> None:
        self._weights.clear()

    # -- reference kernel interface --------------------------------------
    def matmul(self, activation: np.ndarray, tensor_info, weight_bytes) -> np.ndarray:
        """``activation @ W.T`` for ``activation`` [M, K] (numpy) -> float32 [M, N] (numpy)."""
        key = bytes_weight_key(tensor_info, tensor_info.ggml_type, weight_bytes)
        w = self.resident_weight(key, tensor_info, tensor_info.ggml_type, lambda: weight_bytes)
        x = torch.from_numpy(np.ascontiguousarray(activation, dtype=np.float32)).to(self.device)
        return gguf_linear(x, w.data, w.ggml_type, w.shape).cpu().numpy()

    # -- _linear ---------------------------------------------------------
    def linear(self, reader, name: str, x: Array, bias_name: Optional[str] = None) -> Array:
        info, kernel_type, fetch = _describe(reader, name)
        w = self.resident_weight(linear_weight_key(reader, info, kernel_type), info, kernel_type, fetch)
        host = isinstance(x, np.ndarray)
        xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(self.device) if host else x
        bias = self._bias(reader, bias_name) if bias_name is not None and _has_tensor(reader, bias_name) else None
        y = gguf_linear(xd, w.data, w.ggml_type, w.shape, bias=bias)
        return y.cpu().numpy() if host else y

    def _bias(self, reader, name: str) -> torch.Tensor:
        key = ("bias", reader_key(reader), name)
        b = self._weights.get(key)
        if b is None:
            if isinstance(reader, GGUFFile):
                t = reader.tensor(name)
                if t.info.ggml_type != 0:
                    raise KernelError(f"bias '{name}' is not float32")
                arr = np.frombuffer(reader.payload(name), dtype=np.float32)
            else:
                arr = np.asarray(reader.get_tensor(name, dequantize=True), dtype=np.float32).reshape(-1)
            b = torch.from_numpy(arr.copy()).to(self.device)
            self._weights[key] = b
        return b


def _describe(reader, name: str):
    """(tensor info, ggml type for the kernels, payload fetcher) from either reader."""
    if isinstance(reader, GGUFFile):
        t = reader.tensor(name)
        return t.info, t.kernel_type, lambda: reader.payload(name)
    info = reader.tensor_info(name)
    return info, info.ggml_type, lambda: reader._raw_bytes(info.offset, info.nbytes)


def _has_tensor(reader, name: str) -> bool:
    if isinstance(reader, GGUFFile):
        return name in reader.tensor_names()
    return name in getattr(reader, "_index", {})
