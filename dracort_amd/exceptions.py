"""Error classes of the GGUF hot path.

Same names and hierarchy as the reference's ``draco/exceptions.py:6-106`` for
the classes this path raises, so callers that catch the reference's errors
catch these: ``DracoFormatError`` for an unsupported ggml type, a row length
that is not a multiple of the block size or a truncated payload
(``draco/format/gguf.py:284-296``), ``KernelError`` for a kernel that is
unavailable or fails (``draco/exceptions.py:45``), ``KVCacheError`` for a
decode step past the end of its KV cache (``draco/exceptions.py:61``),
``CPUError`` for executor-level errors such as a missing weight tensor
(``draco/exceptions.py:85``).
"""

from __future__ import annotations


class DracoError(Exception):
    """Base error for all Draco exceptions."""


class QuantizationError(DracoError):
    """Raised when quantization operations fail."""


class KernelError(DracoError):
    """Raised when a GPU kernel is unavailable or fails."""


class DracoFormatError(DracoError):
    """Raised when GGUF block data is malformed or of an unsupported type."""


class KVCacheError(DracoError):
    """Raised when the KV cache cannot take another token."""


class CPUError(DracoError):
    """Raised by the executor (name kept from the reference's CPU executor errors)."""
