"""GGUF quantized-matmul operators on MI355X (the ``draco.kernels`` namespace
counterpart for quantized weights).

Every function takes PyTorch-ROCm tensors, checks shapes, dtypes, devices and
buffer sizes on the host, and enqueues the HIP kernels of libdraco_gguf.so on
the current torch stream of the tensors' device.  Nothing here computes on the
CPU and nothing falls back to another implementation: a missing library or a
CPU tensor raises.

Reference call sites replaced:

* ``gguf_dequantize``  ``_dequantize`` + ``GGUFReader.get_tensor``
                       (``draco/format/gguf.py:272-497,820-834``), bit-exact.
* ``gguf_linear``      ``_linear`` (``draco/runtime/cpu/executor.py:47-79``):
                       ``activation.astype(f32) @ W.T (+ bias)``
                       (``draco/runtime/cpu/kernels/generic.py:32-33``) with the
                       dequantization fused into the GEMV (M <= 16) or GEMM.
* ``gguf_moe``         ``TopKRouter.forward`` + ``ExpertGroup.forward``
                       (``draco/models/moe/router.py:81-120``,
                       ``draco/models/moe/expert.py:77-116``).
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from dracort_amd import _native
from dracort_amd.exceptions import DracoFormatError
from dracort_amd.format.gguf import layout, tensor_bytes

GEMV_MAX_M = 16


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need_gpu(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU (got {t.device}); the GGUF path has no CPU implementation")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % 16 != 0:
        raise ValueError(f"{name} must be 16-byte aligned")


def _same_device(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def _check_weight(qweight: torch.Tensor, ggml_type: int, shape: Tuple[int, int]) -> Tuple[int, int]:
    _need_gpu(qweight, "qweight")
    if qweight.dtype != torch.uint8:
        raise ValueError(f"qweight must be uint8 GGUF block bytes, got {qweight.dtype}")
    if len(shape) != 2:
        raise ValueError(f"weight shape must be [N, K], got {shape}")
    n, k = int(shape[0]), int(shape[1])
    need = tensor_bytes(ggml_type, (n, k))
    if qweight.numel() < need:
        raise DracoFormatError(
            f"GGUF payload holds {qweight.numel()} bytes but a {shape} ggml type {ggml_type} tensor needs {need}"
        )
    return n, k


def _x_dtype(x: torch.Tensor) -> int:
    if x.dtype == torch.float32:
        return _native.DRACO_DTYPE_F32
    if x.dtype == torch.bfloat16:
        return _native.DRACO_DTYPE_BF16
    raise ValueError(f"activations must be float32 or bfloat16, got {x.dtype}")


def _flat_bytes(ggml_type: int, n: int, k: int) -> int:
    """Bytes of an [n, k] tensor whose blocks may run across rows (the
    reference's rule: n * k a multiple of the block size)."""
    qk, nb = layout(ggml_type)
    if (n * k) % qk:
        raise DracoFormatError(
            f"GGUF tensor [{n}, {k}] has {n * k} elements, not a multiple of block size {qk} for ggml type {ggml_type}"
        )
    return n * k // qk * nb


def gguf_dequantize(
    qweight: torch.Tensor, ggml_type: int, shape: Tuple[int, int], out: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """float32 [N, K] weight, bit-exact to the reference dequantization.  K
    need not be a multiple of the block size when N * K is (blocks running
    across rows, as ``_dequantize`` allows, ``draco/format/gguf.py:292-296``)."""
    n, k = int(shape[0]), int(shape[1])
    if len(shape) == 2 and k % layout(ggml_type)[0] != 0:
        _need_gpu(qweight, "qweight")
        if qweight.dtype != torch.uint8 or qweight.numel() < _flat_bytes(ggml_type, n, k):
            raise DracoFormatError(f"GGUF payload holds {qweight.numel()} bytes, too few for {tuple(shape)}")
    else:
        n, k = _check_weight(qweight, ggml_type, shape)
    if out is None:
        out = torch.empty((n, k), dtype=torch.float32, device=qweight.device)
    else:
        _need_gpu(out, "out")
        if out.dtype != torch.float32 or out.numel() != n * k:
            raise ValueError(f"out must be float32 with {n * k} elements")
    _same_device(qweight, out)
    lib = _native.load()
    with torch.cuda.device(qweight.device):
        rc = lib.draco_gguf_dequant_f32(
            int(ggml_type), qweight.data_ptr(), qweight.numel(), out.data_ptr(), n, k, _stream(qweight)
        )
    _native.check(rc, "gguf_dequantize")
    return out.view(n, k)


def _prep_linear(x, qweight, ggml_type, shape, bias, out):
    n, k = _check_weight(qweight, ggml_type, shape)
    _need_gpu(x, "x")
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects K={k}")
    m = x.numel() // k if x.numel() else 0
    if m < 1:
        raise ValueError("x holds no rows")
    xd = _x_dtype(x)
    if bias is not None:
        _need_gpu(bias, "bias")
        if bias.dtype != torch.float32 or bias.numel() != n:
            raise ValueError(f"bias must be float32 with {n} elements")
    out_shape = tuple(x.shape[:-1]) + (n,)
    if out is None:
        out = torch.empty(out_shape, dtype=torch.float32, device=x.device)
    else:
        _need_gpu(out, "out")
        if out.dtype != torch.float32 or out.numel() != m * n:
            raise ValueError(f"out must be float32 with {m * n} elements")
    _same_device(x, qweight, out, *( [bias] if bias is not None else []))
    return m, n, k, xd, out


def gemm_workspace_bytes(ggml_type: int, m: int, k: int) -> int:
    """Device workspace bytes the prefill GEMM uses for ``m`` rows of length ``k``."""
    return int(_native.load().draco_gguf_gemm_workspace_size(int(ggml_type), int(m), int(k)))


def _gemm_workspace(ggml_type, m, k, device, workspace):
    need = gemm_workspace_bytes(ggml_type, m, k)
    if need == 0:
        return None, 0
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    _need_gpu(workspace, "workspace")
    if workspace.dtype != torch.uint8:
        raise ValueError("workspace must be a uint8 tensor")
    # a caller's workspace below ``need`` still runs when it holds the required
    # part (the kernels then skip the split-K path); below that the library
    # answers DRACO_EWORKSPACE
    return workspace, workspace.numel()


def gguf_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    ggml_type: int,
    shape: Tuple[int, int],
    bias: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``x @ dequant(W).T (+ bias)`` for x [..., K] (float32 or bfloat16) -> float32 [..., N].

    Prompt-sized bfloat16 inputs take the prefill GEMM, with ``workspace``
    (allocated here when not given) for the types whose GEMM uses one."""
    m, n, k, xd, out = _prep_linear(x, qweight, ggml_type, shape, bias, out)
    ws, ws_bytes = (None, 0)
    if m > GEMV_MAX_M and x.dtype == torch.bfloat16:
        ws, ws_bytes = _gemm_workspace(ggml_type, m, k, x.device, workspace)
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_linear(
            int(ggml_type), qweight.data_ptr(), qweight.numel(), x.data_ptr(), xd,
            bias.data_ptr() if bias is not None else None, out.data_ptr(), m, n, k,
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream(x),
        )
    _native.check(rc, "gguf_linear")
    return out


def gguf_gemv(x, qweight, ggml_type, shape, bias=None, out=None) -> torch.Tensor:
    """Decode GEMV (1..16 activation rows), dequantization fused."""
    m, n, k, xd, out = _prep_linear(x, qweight, ggml_type, shape, bias, out)
    if m > GEMV_MAX_M:
        raise ValueError(f"gguf_gemv takes at most {GEMV_MAX_M} rows, got {m}")
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_gemv(
            int(ggml_type), qweight.data_ptr(), qweight.numel(), x.data_ptr(), xd,
            bias.data_ptr() if bias is not None else None, out.data_ptr(), m, n, k, _stream(x),
        )
    _native.check(rc, "gguf_gemv")
    return out


def gguf_gemm(x, qweight, ggml_type, shape, bias=None, out=None, workspace=None) -> torch.Tensor:
    """Prefill GEMM (bf16 activations, MFMA), dequantization fused.  ``workspace``
    (uint8 device tensor of ``gemm_workspace_bytes`` bytes) is allocated here
    when not given."""
    if x.dtype != torch.bfloat16:
        raise ValueError(f"gguf_gemm takes bfloat16 activations, got {x.dtype}")
    m, n, k, xd, out = _prep_linear(x, qweight, ggml_type, shape, bias, out)
    ws, ws_bytes = _gemm_workspace(ggml_type, m, k, x.device, workspace)
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_gemm(
            int(ggml_type), qweight.data_ptr(), qweight.numel(), x.data_ptr(),
            bias.data_ptr() if bias is not None else None, out.data_ptr(), m, n, k,
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream(x),
        )
    _native.check(rc, "gguf_gemm")
    return out


def _out_check(t: Optional[torch.Tensor], dtype, numel: int, name: str) -> None:
    if t is None:
        return
    _need_gpu(t, name)
    if t.dtype != dtype or t.numel() != numel:
        raise ValueError(f"{name} must be {dtype} with {numel} elements")


def _x_rows(x: torch.Tensor, k: int) -> int:
    _need_gpu(x, "x")
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects K={k}")
    m = x.numel() // k
    if not 1 <= m <= GEMV_MAX_M:
        raise ValueError(f"fused GEMVs take 1..{GEMV_MAX_M} activation rows, got {m}")
    return m


def gguf_gemv_multi(
    x: torch.Tensor,
    weights: Sequence[Tuple[torch.Tensor, int]],
    ggml_type: int,
    k: int,
    outs: Sequence[Optional[torch.Tensor]],
    outs_bf16: Optional[Sequence[Optional[torch.Tensor]]] = None,
) -> None:
    """One launch for several [n_i, K] weights sharing x (e.g. q, k, v).

    ``weights`` = [(qweight_i, n_i)]; ``outs[i]`` float32 [m, n_i] and/or
    ``outs_bf16[i]`` bfloat16 [m, n_i] (either may be None).
    """
    m = _x_rows(x, k)
    nm = len(weights)
    if not 1 <= nm <= 4 or len(outs) != nm or (outs_bf16 is not None and len(outs_bf16) != nm):
        raise ValueError("1..4 weights with one output slot each")
    outs_bf16 = list(outs_bf16) if outs_bf16 is not None else [None] * nm
    for i, (q, n) in enumerate(weights):
        _check_weight(q, ggml_type, (n, k))
        _same_device(x, q)
        if outs[i] is None and outs_bf16[i] is None:
            raise ValueError(f"weight {i} has no output")
        _out_check(outs[i], torch.float32, m * n, f"outs[{i}]")
        _out_check(outs_bf16[i], torch.bfloat16, m * n, f"outs_bf16[{i}]")
    vp = ctypes.c_void_p
    w_arr = (vp * nm)(*[q.data_ptr() for q, _ in weights])
    b_arr = (ctypes.c_size_t * nm)(*[q.numel() for q, _ in weights])
    n_arr = (ctypes.c_int64 * nm)(*[int(n) for _, n in weights])
    y_arr = (vp * nm)(*[o.data_ptr() if o is not None else None for o in outs])
    yb_arr = (vp * nm)(*[o.data_ptr() if o is not None else None for o in outs_bf16])
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_gemv_multi(int(ggml_type), nm, w_arr, b_arr, n_arr, y_arr, yb_arr, x.data_ptr(),
                                       _x_dtype(x), m, k, _stream(x))
    _native.check(rc, "gguf_gemv_multi")


def gguf_gemv_swiglu(
    x: torch.Tensor,
    w_gate: torch.Tensor,
    w_up: torch.Tensor,
    ggml_type: int,
    shape: Tuple[int, int],
    out: Optional[torch.Tensor] = None,
    out_bf16: Optional[torch.Tensor] = None,
) -> None:
    """silu(x @ W_gate.T) * (x @ W_up.T) into float32 ``out`` and/or bfloat16 ``out_bf16``."""
    n, k = _check_weight(w_gate, ggml_type, shape)
    _check_weight(w_up, ggml_type, shape)
    if w_gate.numel() != w_up.numel():
        raise ValueError("gate and up buffers differ in size")
    m = _x_rows(x, k)
    if out is None and out_bf16 is None:
        raise ValueError("need out and/or out_bf16")
    _out_check(out, torch.float32, m * n, "out")
    _out_check(out_bf16, torch.bfloat16, m * n, "out_bf16")
    _same_device(x, w_gate, w_up)
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_gemv_swiglu(
            int(ggml_type), w_gate.data_ptr(), w_up.data_ptr(), w_gate.numel(), x.data_ptr(), _x_dtype(x),
            out.data_ptr() if out is not None else None, out_bf16.data_ptr() if out_bf16 is not None else None,
            m, n, k, _stream(x),
        )
    _native.check(rc, "gguf_gemv_swiglu")


def gguf_gemv_residual(
    x: torch.Tensor,
    qweight: torch.Tensor,
    ggml_type: int,
    shape: Tuple[int, int],
    resid: torch.Tensor,
    resid_bf16: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> None:
    """resid += x @ W.T in place (float32); resid_bf16 = bf16(resid) if given.
    ``workspace`` (uint8 device tensor of ``gemv_residual_workspace_bytes``
    bytes, or None) lets launches with few tiles and long rows split K."""
    n, k = _check_weight(qweight, ggml_type, shape)
    m = _x_rows(x, k)
    _out_check(resid, torch.float32, m * n, "resid")
    _out_check(resid_bf16, torch.bfloat16, m * n, "resid_bf16")
    _same_device(x, qweight, resid)
    lib = _native.load()
    rb = resid_bf16.data_ptr() if resid_bf16 is not None else None
    with torch.cuda.device(x.device):
        if workspace is None:
            rc = lib.draco_gguf_gemv_residual(
                int(ggml_type), qweight.data_ptr(), qweight.numel(), x.data_ptr(), _x_dtype(x), resid.data_ptr(),
                rb, m, n, k, _stream(x),
            )
        else:
            _need_gpu(workspace, "workspace")
            if workspace.dtype != torch.uint8:
                raise ValueError("workspace must be a uint8 tensor")
            rc = lib.draco_gguf_gemv_residual_ws(
                int(ggml_type), qweight.data_ptr(), qweight.numel(), x.data_ptr(), _x_dtype(x), resid.data_ptr(),
                rb, m, n, k, workspace.data_ptr(), workspace.numel(), _stream(x),
            )
    _native.check(rc, "gguf_gemv_residual")


def gemv_residual_workspace_bytes(ggml_type: int, m: int, n: int, k: int) -> int:
    """Bytes of split-K workspace gguf_gemv_residual uses for this launch (0: none)."""
    return int(_native.load().draco_gguf_gemv_residual_workspace_size(int(ggml_type), int(m), int(n), int(k)))


def _norm_args(x: torch.Tensor, norm_weight: torch.Tensor, x_norm: torch.Tensor, k: int) -> int:
    _need_gpu(x, "x")
    _need_gpu(norm_weight, "norm_weight")
    _need_gpu(x_norm, "x_norm")
    if x.dtype != torch.float32 or norm_weight.dtype != torch.float32:
        raise ValueError("fused RMSNorm takes float32 x and norm_weight")
    if x.numel() % k or tuple(norm_weight.shape) != (k,):
        raise ValueError(f"x must be [m, {k}] and norm_weight [{k}]")
    m = x.numel() // k
    if x_norm.dtype != torch.bfloat16 or x_norm.numel() != m * k:
        raise ValueError(f"x_norm must be bfloat16 [{m}, {k}]")
    _same_device(x, norm_weight, x_norm)
    return m


def gguf_gemv_multi_rmsnorm(
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float,
    x_norm: torch.Tensor,
    weights: Sequence[Tuple[torch.Tensor, int]],
    ggml_type: int,
    k: int,
    outs: Sequence[Optional[torch.Tensor]],
    outs_bf16: Optional[Sequence[Optional[torch.Tensor]]] = None,
) -> None:
    """``gguf_gemv_multi`` on ``x_norm = bf16(rms_norm(x, norm_weight, eps))`` (x float32
    [m, k]; x_norm is written).  The norm runs in the GEMV's prologue where the
    persistent single-token kernel applies, else as its own launch."""
    m = _norm_args(x, norm_weight, x_norm, k)
    nm = len(weights)
    if not 1 <= nm <= 4 or len(outs) != nm or (outs_bf16 is not None and len(outs_bf16) != nm):
        raise ValueError("1..4 weights with one output slot each")
    outs_bf16 = list(outs_bf16) if outs_bf16 is not None else [None] * nm
    for i, (q, n) in enumerate(weights):
        _check_weight(q, ggml_type, (n, k))
        _same_device(x, q)
        if outs[i] is None and outs_bf16[i] is None:
            raise ValueError(f"weight {i} has no output")
        _out_check(outs[i], torch.float32, m * n, f"outs[{i}]")
        _out_check(outs_bf16[i], torch.bfloat16, m * n, f"outs_bf16[{i}]")
    vp = ctypes.c_void_p
    w_arr = (vp * nm)(*[q.data_ptr() for q, _ in weights])
    b_arr = (ctypes.c_size_t * nm)(*[q.numel() for q, _ in weights])
    n_arr = (ctypes.c_int64 * nm)(*[int(n) for _, n in weights])
    y_arr = (vp * nm)(*[o.data_ptr() if o is not None else None for o in outs])
    yb_arr = (vp * nm)(*[o.data_ptr() if o is not None else None for o in outs_bf16])
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_gemv_multi_rmsnorm(int(ggml_type), nm, w_arr, b_arr, n_arr, y_arr, yb_arr, x.data_ptr(),
                                               norm_weight.data_ptr(), float(eps), x_norm.data_ptr(), m, k,
                                               _stream(x))
    _native.check(rc, "gguf_gemv_multi_rmsnorm")


def gguf_gemv_swiglu_rmsnorm(
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float,
    x_norm: torch.Tensor,
    w_gate: torch.Tensor,
    w_up: torch.Tensor,
    ggml_type: int,
    shape: Tuple[int, int],
    out: Optional[torch.Tensor] = None,
    out_bf16: Optional[torch.Tensor] = None,
) -> None:
    """``gguf_gemv_swiglu`` on ``x_norm = bf16(rms_norm(x, norm_weight, eps))``."""
    n, k = _check_weight(w_gate, ggml_type, shape)
    _check_weight(w_up, ggml_type, shape)
    if w_gate.numel() != w_up.numel():
        raise ValueError("gate and up buffers differ in size")
    m = _norm_args(x, norm_weight, x_norm, k)
    if out is None and out_bf16 is None:
        raise ValueError("need out and/or out_bf16")
    _out_check(out, torch.float32, m * n, "out")
    _out_check(out_bf16, torch.bfloat16, m * n, "out_bf16")
    _same_device(x, w_gate, w_up)
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_gemv_swiglu_rmsnorm(
            int(ggml_type), w_gate.data_ptr(), w_up.data_ptr(), w_gate.numel(), x.data_ptr(), norm_weight.data_ptr(),
            float(eps), x_norm.data_ptr(), out.data_ptr() if out is not None else None,
            out_bf16.data_ptr() if out_bf16 is not None else None, m, n, k, _stream(x))
    _native.check(rc, "gguf_gemv_swiglu_rmsnorm")


def moe_workspace_bytes(tokens: int, hidden: int, inter: int, n_experts: int, top_k: int) -> int:
    return int(_native.load().draco_gguf_moe_workspace_size(tokens, hidden, inter, n_experts, top_k))


def gguf_moe(
    x: torch.Tensor,
    router_logits: torch.Tensor,
    w_gate: Sequence[torch.Tensor],
    w_up: Sequence[torch.Tensor],
    w_down: Sequence[torch.Tensor],
    ggml_type: int,
    inter: int,
    top_k: int = 2,
    workspace: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Sparse MoE FFN: top-k softmax routing + per-expert GGUF SwiGLU FFN.

    x [T, H] (float32/bfloat16), router_logits [T, E] float32, w_gate[e] /
    w_up[e] GGUF [inter, H], w_down[e] GGUF [H, inter]; returns float32 [T, H].
    """
    _need_gpu(x, "x")
    _need_gpu(router_logits, "router_logits")
    if x.dim() != 2:
        raise ValueError("x must be [tokens, hidden]")
    t, h = x.shape
    e = len(w_gate)
    if not (len(w_up) == e and len(w_down) == e and e >= 1):
        raise ValueError("w_gate, w_up and w_down must list the same experts")
    if router_logits.dtype != torch.float32 or tuple(router_logits.shape) != (t, e):
        raise ValueError(f"router_logits must be float32 [{t}, {e}]")
    xd = _x_dtype(x)
    need = tensor_bytes(ggml_type, (inter, h))
    if tensor_bytes(ggml_type, (h, inter)) != need:
        raise DracoFormatError("gate/up and down expert shapes disagree")
    for name, ws in (("w_gate", w_gate), ("w_up", w_up), ("w_down", w_down)):
        for i, w in enumerate(ws):
            _need_gpu(w, f"{name}[{i}]")
            if w.dtype != torch.uint8 or w.numel() < need:
                raise DracoFormatError(f"{name}[{i}] must be uint8 GGUF blocks of >= {need} bytes")
            _same_device(x, w)
    ws_bytes = moe_workspace_bytes(t, h, inter, e, top_k)
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    else:
        _need_gpu(workspace, "workspace")
    if out is None:
        out = torch.empty((t, h), dtype=torch.float32, device=x.device)
    else:
        _need_gpu(out, "out")
        if out.dtype != torch.float32 or out.numel() != t * h:
            raise ValueError(f"out must be float32 with {t * h} elements")
    _same_device(x, router_logits, workspace, out)
    arr = ctypes.c_void_p * e
    pg = arr(*[w.data_ptr() for w in w_gate])
    pu = arr(*[w.data_ptr() for w in w_up])
    pd = arr(*[w.data_ptr() for w in w_down])
    lib = _native.load()
    with torch.cuda.device(x.device):
        rc = lib.draco_gguf_moe_ffn(
            int(ggml_type), pg, pu, pd, need, router_logits.data_ptr(), x.data_ptr(), xd, out.data_ptr(),
            t, h, int(inter), e, int(top_k), workspace.data_ptr(), workspace.numel(), _stream(x),
        )
    _native.check(rc, "gguf_moe")
    return out


def block_layout(ggml_type: int) -> Tuple[int, int]:
    """(elements, bytes) per block, from the library (checks it loads)."""
    host = layout(ggml_type)
    dev = _native.block_info(ggml_type)
    if host != dev:
        raise DracoFormatError(f"block layout mismatch for type {ggml_type}: {host} vs library {dev}")
    return dev
