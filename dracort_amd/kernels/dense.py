"""Executor operators for the GGUF tensors that are not block-quantized, and
the glue between projections that were not fused into one launch.

Reference call sites replaced:

* ``dense_linear``  ``_linear`` on a tensor with ``quantization=None``:
                    ``get_tensor(dequantize=True)`` then ``matmul_f32`` =
                    ``x.astype(f32) @ W.T (+ bias)``
                    (``draco/runtime/cpu/executor.py:47-52,77-78``,
                    ``draco/runtime/cpu/kernels/generic.py:32-33``) for
                    F32 / F16 / BF16 weights; ``accumulate=True`` adds the
                    product into ``out`` (the residual add of ``forward_step``).
* ``get_rows``      ``embed[token_ids]`` of ``_initial_hidden``
                    (``draco/runtime/cpu/executor.py:279-288``) for float or
                    block-quantized tables (bit-exact dequantization).
* ``swiglu``        ``swiglu`` (``draco/runtime/cpu/ops.py:19-27``) of gate /
                    up projections computed by separate launches.

Everything runs through libdraco_gguf.so on the GPU; CPU tensors raise.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from dracort_amd import _native
from dracort_amd.exceptions import DracoFormatError
from dracort_amd.format.gguf import BLOCK_LAYOUTS, base_type, tensor_bytes
from dracort_amd.kernels.gguf import _need_gpu, _same_device, _stream, _x_dtype

# ggml float types the dense kernels read: id -> (name, bytes per element)
FLOAT_TYPES = {0: ("f32", 4), 1: ("f16", 2), 30: ("bf16", 2)}


def _ptr_ok(t: torch.Tensor, name: str, align: int) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor; the GGUF path has no CPU implementation")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")


def dense_linear(x: torch.Tensor, weight: torch.Tensor, ggml_type: int, shape: Tuple[int, int],
                 bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                 accumulate: bool = False) -> torch.Tensor:
    """``x @ W.T (+ bias)`` for a float weight (``weight``: its raw bytes as a
    uint8 tensor, or a float32 / float16 / bfloat16 tensor) -> float32
    [..., N]; with ``accumulate`` the product is added into ``out``."""
    if ggml_type not in FLOAT_TYPES:
        raise DracoFormatError(f"dense_linear takes ggml types F32 / F16 / BF16, got {ggml_type}")
    n, k = int(shape[0]), int(shape[1])
    elem = FLOAT_TYPES[ggml_type][1]
    _ptr_ok(weight, "weight", elem)
    wbytes = weight.numel() * weight.element_size()
    if wbytes < n * k * elem:
        raise DracoFormatError(f"weight holds {wbytes} bytes, [{n}, {k}] of ggml type {ggml_type} needs {n * k * elem}")
    _ptr_ok(x, "x", x.element_size())
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects K={k}")
    m = x.numel() // k
    xd = _x_dtype(x)
    if bias is not None:
        _ptr_ok(bias, "bias", 4)
        if bias.dtype != torch.float32 or bias.numel() != n:
            raise ValueError(f"bias must be float32 with {n} elements")
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = torch.empty(tuple(x.shape[:-1]) + (n,), dtype=torch.float32, device=x.device)
    _ptr_ok(out, "out", 4)
    if out.dtype != torch.float32 or out.numel() != m * n:
        raise ValueError(f"out must be float32 with {m * n} elements")
    _same_device(x, weight, out, *([bias] if bias is not None else []))
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_dense_linear(int(ggml_type), weight.data_ptr(), wbytes, x.data_ptr(), xd,
                                         bias.data_ptr() if bias is not None else None, out.data_ptr(), m, n, k,
                                         1 if accumulate else 0, _stream(x))
    _native.check(rc, "dense_linear")
    return out


def get_rows(table: torch.Tensor, ggml_type: int, shape: Tuple[int, int], ids: torch.Tensor,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """float32 [len(ids), K] = rows ``ids`` (int32, on the device) of the
    [N, K] table (raw bytes as uint8, block-quantized or float); an id
    outside [0, N) gives a NaN row."""
    n, k = int(shape[0]), int(shape[1])
    base = base_type(ggml_type)
    if base in FLOAT_TYPES:
        need, align = n * k * FLOAT_TYPES[base][1], FLOAT_TYPES[base][1]
    elif base in BLOCK_LAYOUTS:
        need, align = tensor_bytes(ggml_type, (n, k)), 16
    else:
        raise DracoFormatError(f"get_rows: unsupported ggml type {ggml_type}")
    _ptr_ok(table, "table", align)
    nbytes = table.numel() * table.element_size()
    if nbytes < need:
        raise DracoFormatError(f"table holds {nbytes} bytes, [{n}, {k}] of ggml type {ggml_type} needs {need}")
    _need_gpu(ids, "ids")
    if ids.dtype != torch.int32:
        raise ValueError("ids must be int32")
    t = ids.numel()
    if out is None:
        out = torch.empty((t, k), dtype=torch.float32, device=table.device)
    _ptr_ok(out, "out", 16 if base not in FLOAT_TYPES else 4)
    if out.dtype != torch.float32 or out.numel() != t * k:
        raise ValueError(f"out must be float32 [{t}, {k}]")
    _same_device(table, ids, out)
    lib = _native.load()
    with torch.cuda.device(table.device):
        rc = lib.draco_gguf_get_rows(int(ggml_type), table.data_ptr(), nbytes, n, k, ids.data_ptr(), t,
                                     out.data_ptr(), _stream(table))
    _native.check(rc, "get_rows")
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: Optional[torch.Tensor] = None,
           out_bf16: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(gate) * up (float32 in) into float32 ``out`` and / or bfloat16 ``out_bf16``."""
    for t, name in ((gate, "gate"), (up, "up")):
        _ptr_ok(t, name, 4)
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be float32")
    if gate.shape != up.shape:
        raise ValueError("gate and up differ in shape")
    n = gate.numel()
    if out is None and out_bf16 is None:
        out = torch.empty_like(gate)
    for t, dt, name in ((out, torch.float32, "out"), (out_bf16, torch.bfloat16, "out_bf16")):
        if t is not None:
            _ptr_ok(t, name, t.element_size())
            if t.dtype != dt or t.numel() != n:
                raise ValueError(f"{name} must be {dt} with {n} elements")
    _same_device(gate, up, *[t for t in (out, out_bf16) if t is not None])
    lib = _native.load()
    with torch.cuda.device(gate.device):
        rc = lib.draco_gguf_swiglu(gate.data_ptr(), up.data_ptr(), out.data_ptr() if out is not None else None,
                                   out_bf16.data_ptr() if out_bf16 is not None else None, n, _stream(gate))
    _native.check(rc, "swiglu")
    return out if out is not None else out_bf16
