"""ctypes binding of libdraco_gguf.so (C ABI declared in include/draco_gguf.h).

The library is built in-tree (``make -C dracort_amd/csrc``, or
``__graft_entry__.build()``) into ``dracort_amd/lib/libdraco_gguf.so``.  There
is no fallback: if the library is missing or fails to load, every operator
raises :class:`KernelError`.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

from dracort_amd.exceptions import DracoFormatError, KernelError

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libdraco_gguf.so")

# return codes (include/draco_gguf.h)
DRACO_OK = 0
DRACO_EINVAL_QTYPE = -1
DRACO_EINVAL_SHAPE = -2
DRACO_EINVAL_ARG = -3
DRACO_EHIP = -4
DRACO_EWORKSPACE = -5

DRACO_DTYPE_F32 = 0
DRACO_DTYPE_BF16 = 1
DRACO_GGUF_GGML_ORDER = 0x100  # Q2_K / Q3_K / Q6_K in upstream ggml field order
DRACO_GGUF_Q6K_D_LAST = DRACO_GGUF_GGML_ORDER
DRACO_GGUF_NOALLOC_SCRATCH_BYTES = 64 << 20

ABI_VERSION = 4

_c_int, _c_i64, _c_size, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); every symbol the header declares
SIGNATURES = {
    "draco_gguf_abi_version": (_c_int, []),
    "draco_gguf_last_error": (ctypes.c_char_p, []),
    "draco_gguf_block_info": (_c_int, [_c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)]),
    "draco_gguf_dequant_f32": (_c_int, [_c_int, _vp, _c_size, _vp, _c_i64, _c_i64, _vp]),
    "draco_gguf_gemv": (_c_int, [_c_int, _vp, _c_size, _vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "draco_gguf_gemv_multi": (
        _c_int,
        [_c_int, _c_int, ctypes.POINTER(_vp), ctypes.POINTER(_c_size), ctypes.POINTER(_c_i64), ctypes.POINTER(_vp),
         ctypes.POINTER(_vp), _vp, _c_int, _c_i64, _c_i64, _vp],
    ),
    "draco_gguf_gemv_swiglu": (_c_int, [_c_int, _vp, _vp, _c_size, _vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "draco_gguf_gemv_residual": (_c_int, [_c_int, _vp, _c_size, _vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "draco_gguf_gemv_residual_workspace_size": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64]),
    "draco_gguf_gemv_residual_ws": (_c_int, [_c_int, _vp, _c_size, _vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                             _vp, _c_size, _vp]),
    "draco_gguf_gemm_workspace_size": (_c_size, [_c_int, _c_i64, _c_i64]),
    "draco_gguf_gemm": (_c_int, [_c_int, _vp, _c_size, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_size, _vp]),
    "draco_gguf_linear": (
        _c_int, [_c_int, _vp, _c_size, _vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_size, _vp]
    ),
    "draco_gguf_linear_noalloc": (
        _c_int, [_c_int, _vp, _c_size, _vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]
    ),
    "draco_gguf_moe_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "draco_gguf_moe_ffn": (
        _c_int,
        [_c_int, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp), _c_size, _vp, _vp, _c_int, _vp,
         _c_i64, _c_i64, _c_i64, _c_int, _c_int, _vp, _c_size, _vp],
    ),
    "draco_gguf_gemv_multi_rmsnorm": (
        _c_int,
        [_c_int, _c_int, ctypes.POINTER(_vp), ctypes.POINTER(_c_size), ctypes.POINTER(_c_i64), ctypes.POINTER(_vp),
         ctypes.POINTER(_vp), _vp, _vp, ctypes.c_float, _vp, _c_i64, _c_i64, _vp],
    ),
    "draco_gguf_gemv_swiglu_rmsnorm": (
        _c_int, [_c_int, _vp, _vp, _c_size, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]
    ),
    "draco_gguf_rms_norm": (_c_int, [_vp, _vp, ctypes.c_float, _vp, _vp, _c_i64, _c_i64, _vp]),
    "draco_gguf_decode_attention_workspace_size": (_c_size, [_c_i64, _c_int, _c_int, _c_int, _c_i64]),
    "draco_gguf_decode_attention": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_int, _c_int, _c_int, _c_i64, _vp, _vp, _vp, _c_int, _vp, _c_size,
         _vp],
    ),
    "draco_gguf_dense_linear": (
        _c_int, [_c_int, _vp, _c_size, _vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_int, _vp]
    ),
    "draco_gguf_get_rows": (_c_int, [_c_int, _vp, _c_size, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    "draco_gguf_swiglu": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _vp]),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def load(path: Optional[str] = None) -> ctypes.CDLL:
    """Load (once) and return the library with argtypes/restypes installed."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise KernelError(
                f"libdraco_gguf.so not found at {p}; build it with "
                f"`make -C dracort_amd/csrc` (or __graft_entry__.build())."
            )
        try:
            lib = ctypes.CDLL(p)
        except OSError as exc:
            raise KernelError(f"failed to load {p}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.draco_gguf_abi_version()
        if ver != ABI_VERSION:
            raise KernelError(f"{p} has ABI version {ver}, this package expects {ABI_VERSION}; rebuild it.")
        if path is None:
            _lib = lib
        return lib


def last_error() -> str:
    msg = load().draco_gguf_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Map a DRACO_E* return code onto the reference's exception classes."""
    if rc == DRACO_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc in (DRACO_EINVAL_QTYPE, DRACO_EINVAL_SHAPE):
        raise DracoFormatError(msg)
    if rc == DRACO_EINVAL_ARG:
        raise ValueError(msg)
    raise KernelError(f"{msg} (code {rc})")


def block_info(ggml_type: int):
    qk, nb = _c_int(0), _c_int(0)
    check(load().draco_gguf_block_info(int(ggml_type), ctypes.byref(qk), ctypes.byref(nb)), "block_info")
    return qk.value, nb.value
