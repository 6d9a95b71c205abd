"""Decode-step glue operators on MI355X: RMSNorm and single-token attention
over a float16 KV cache (RoPE and the cache append fused in).

Reference call sites replaced:

* ``rms_norm``          ``rms_norm`` (``draco/runtime/cpu/ops.py:15-19``) as
                        ``_norm`` calls it (``draco/runtime/cpu/executor.py:199-206``);
                        also ``fused_rms_norm`` (``draco/kernels/ops.py:29-52``).
* ``decode_attention``  ``apply_rope`` on q / k (``draco/runtime/cpu/ops.py:73-92``),
                        ``CPUKVCache.append`` (float16 storage,
                        ``draco/runtime/cpu/kv_cache.py:19-28``) and
                        ``CPUAttentionBackend.decode`` (``draco/runtime/cpu/attention.py:35-81``).

As for the GEMV operators, everything runs on the GPU through
libdraco_gguf.so; CPU tensors or a missing library raise.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch

from dracort_amd import _native
from dracort_amd.kernels.gguf import _need_gpu, _same_device, _stream


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, out: Optional[torch.Tensor] = None,
             out_bf16: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x [m, n] float32, weight [n] float32 -> float32 ``out`` and / or bfloat16
    ``out_bf16`` (float32 ``out`` allocated when neither is given); returns the
    first given output."""
    _need_gpu(x, "x")
    _need_gpu(weight, "weight")
    if x.dtype != torch.float32 or weight.dtype != torch.float32:
        raise ValueError("rms_norm takes float32 x and weight")
    if x.dim() == 1:
        x = x.unsqueeze(0)
    m, n = x.shape
    if tuple(weight.shape) != (n,):
        raise ValueError(f"weight must be [{n}], got {tuple(weight.shape)}")
    if out is None and out_bf16 is None:
        out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    for t, dt, name in ((out, torch.float32, "out"), (out_bf16, torch.bfloat16, "out_bf16")):
        if t is not None:
            _need_gpu(t, name)
            if t.dtype != dt or t.numel() != m * n:
                raise ValueError(f"{name} must be {dt} with {m * n} elements")
            _same_device(x, t)
    _same_device(x, weight)
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_rms_norm(x.data_ptr(), weight.data_ptr(), float(eps),
                                     out.data_ptr() if out is not None else None,
                                     out_bf16.data_ptr() if out_bf16 is not None else None, m, n, _stream(x))
    _native.check(rc, "rms_norm")
    return out if out is not None else out_bf16


def decode_attention_workspace_bytes(batch: int, n_q_heads: int, n_kv_heads: int, head_dim: int,
                                     max_positions: int) -> int:
    return int(_native.load().draco_gguf_decode_attention_workspace_size(batch, n_q_heads, n_kv_heads, head_dim,
                                                                          max_positions))


class DecodeAttentionWorkspace:
    """Device workspace of the decode attention: the partial softmax states
    of its position splits (reused by every call of the same sizes)."""

    def __init__(self, batch: int, n_q_heads: int, n_kv_heads: int, head_dim: int, max_positions: int,
                 device="cuda") -> None:
        nbytes = decode_attention_workspace_bytes(batch, n_q_heads, n_kv_heads, head_dim, max_positions)
        if nbytes == 0:
            raise ValueError("invalid decode attention sizes")
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        self.sizes = (batch, n_q_heads, n_kv_heads, head_dim, max_positions)


def rope_tables(head_dim: int, max_positions: int, theta: float = 10000.0,
                device="cuda") -> Tuple[torch.Tensor, torch.Tensor]:
    """cos / sin [max_positions, head_dim // 2] float32 on the device, built as
    the reference's ``build_rope_cache`` builds them
    (``draco/runtime/cpu/ops.py:73-79``): ``inv_freq = 1 / theta **
    (arange(0, D, 2) / D)``, angles ``position * inv_freq``, all in float32.
    Host-side setup, once per model; the kernels only read the tables."""
    exponent = np.arange(0, head_dim, 2, dtype=np.float32) / head_dim
    inv_freq = 1.0 / (theta ** exponent)
    angles = np.outer(np.arange(max_positions, dtype=np.float32), inv_freq)
    return (torch.from_numpy(np.cos(angles)).to(device), torch.from_numpy(np.sin(angles)).to(device))


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                     v_cache: torch.Tensor, positions: torch.Tensor, n_q_heads: int, n_kv_heads: int,
                     rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, out: Optional[torch.Tensor] = None,
                     out_dtype: torch.dtype = torch.float32,
                     workspace: Optional[DecodeAttentionWorkspace] = None) -> torch.Tensor:
    """One decode token per sequence.

    q [B, n_q_heads * D], k / v [B, n_kv_heads * D] float32 (before RoPE);
    k_cache / v_cache float16 [B, n_kv_heads, max_positions, D]; positions [B]
    int32 on the device (the new token's position = tokens already cached);
    ``rope`` = (cos, sin) tables from :func:`rope_tables` (None: no RoPE).
    Stores the rotated k and v at their position and returns the attention
    output [B, n_q_heads * D] (float32 or bfloat16)."""
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache"),
                    (positions, "positions")):
        _need_gpu(t, name)
    if k_cache.dim() != 4 or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError("k_cache and v_cache must be [B, n_kv_heads, max_positions, head_dim]")
    b, hkv, max_pos, d = k_cache.shape
    if hkv != n_kv_heads:
        raise ValueError(f"k_cache holds {hkv} kv heads, expected {n_kv_heads}")
    if k_cache.dtype != torch.float16 or v_cache.dtype != torch.float16:
        raise ValueError("the KV caches are float16")
    for t, cols, name in ((q, n_q_heads * d, "q"), (k, n_kv_heads * d, "k"), (v, n_kv_heads * d, "v")):
        if t.dtype != torch.float32 or t.numel() != b * cols:
            raise ValueError(f"{name} must be float32 [{b}, {cols}]")
    if positions.dtype != torch.int32 or positions.numel() != b:
        raise ValueError(f"positions must be int32 [{b}]")
    cos_p = sin_p = None
    if rope is not None:
        cos_t, sin_t = rope
        for t, name in ((cos_t, "rope cos"), (sin_t, "rope sin")):
            _need_gpu(t, name)
            if t.dtype != torch.float32 or tuple(t.shape) != (max_pos, d // 2):
                raise ValueError(f"{name} table must be float32 [{max_pos}, {d // 2}]")
            _same_device(q, t)
        cos_p, sin_p = cos_t.data_ptr(), sin_t.data_ptr()
    if out is None:
        out = torch.empty((b, n_q_heads * d), dtype=out_dtype, device=q.device)
    _need_gpu(out, "out")
    if out.dtype not in (torch.float32, torch.bfloat16) or out.numel() != b * n_q_heads * d:
        raise ValueError(f"out must be float32 or bfloat16 [{b}, {n_q_heads * d}]")
    if workspace is None:
        workspace = DecodeAttentionWorkspace(b, n_q_heads, n_kv_heads, d, max_pos, q.device)
    elif workspace.sizes != (b, n_q_heads, n_kv_heads, d, max_pos):
        raise ValueError(f"workspace was made for {workspace.sizes}")
    _same_device(q, k, v, k_cache, v_cache, positions, out, workspace.buf)
    lib = _native.load()
    with torch.cuda.device(q.device):
        rc = lib.draco_gguf_decode_attention(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), positions.data_ptr(),
            b, n_q_heads, n_kv_heads, d, max_pos, cos_p, sin_p, out.data_ptr(),
            _native.DRACO_DTYPE_BF16 if out.dtype == torch.bfloat16 else _native.DRACO_DTYPE_F32,
            workspace.buf.data_ptr(), workspace.buf.numel(), _stream(q))
    _native.check(rc, "decode_attention")
    return out
