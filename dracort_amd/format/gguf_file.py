"""Memory-mapped GGUF container: metadata, tensor directory and zero-copy
access to each tensor's packed blocks.

Follows the container rules the reference's ``GGUFReader`` reads
(``draco/format/gguf.py:527-600``): little-endian header ``"GGUF"``, u32
version (1..3), u64 tensor count, u64 metadata count; metadata as (string
key, u32 value type, value) with arrays as (u32 element type, u64 length,
elements); tensor infos as (string name, u32 n_dims, u64 dims[n_dims], u32
ggml type, u64 offset relative to the data section); the data section
starts at the next multiple of ``general.alignment`` (default 32, a positive
multiple of 8); a tensor's numpy shape is its GGUF dims reversed.  Value
type ids and block sizes are the format's (``draco/format/gguf.py:55-96``).

Unlike the reference, which copies a tensor region to ``bytes`` and
dequantizes it to float32 on first use (``draco/format/gguf.py:812-834``),
this reader hands out the packed payload itself -- a read-only view of the
mapping -- so the uploader can stream it into HBM in its native layout.

Field order.  The reference decodes Q2_K, Q3_K and Q6_K blocks with their
float16 scales first (``draco/format/gguf.py:355-359, 376-380, 470-474``);
upstream ggml files store them last.  ``field_order="reference"`` (default)
reads blocks as the reference does; ``field_order="ggml"`` tags Q2_K / Q3_K /
Q6_K tensors with the kernels' ``GGML_ORDER`` layout flag instead.
"""

from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from typing import Any, Dict, Iterator, List, Optional, Tuple

import numpy as np

from dracort_amd.exceptions import DracoFormatError
from dracort_amd.format.gguf import GGML_ORDER, ORDER_TYPES, GgufTensorInfo

GGUF_MAGIC = b"GGUF"

# ggml tensor types: float types by element size, block types by (elements, bytes)
FLOAT_TYPES = {0: ("f32", 4), 1: ("f16", 2), 28: ("f64", 8), 30: ("bf16", 2)}
BLOCK_TYPES = {
    2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 15: (256, 258),
    10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
}

# metadata value types: id -> (struct code, size); 7 = bool, 8 = string, 9 = array
_SCALARS = {0: ("B", 1), 1: ("b", 1), 2: ("H", 2), 3: ("h", 2), 4: ("I", 4), 5: ("i", 4), 6: ("f", 4),
            7: ("?", 1), 10: ("Q", 8), 11: ("q", 8), 12: ("d", 8)}
_STRING, _ARRAY = 8, 9


class _Cursor:
    """Bounds-checked little-endian reader over the mapped header region."""

    def __init__(self, buf, pos: int, what: str) -> None:
        self.buf, self.pos, self.what = buf, pos, what

    def take(self, n: int) -> memoryview:
        if n < 0 or self.pos + n > len(self.buf):
            raise DracoFormatError(f"GGUF {self.what}: field at byte {self.pos} runs past the end of the file.")
        v = self.buf[self.pos:self.pos + n]
        self.pos += n
        return v

    def unpack(self, code: str, size: int):
        return struct.unpack("<" + code, self.take(size))[0]

    def u32(self) -> int:
        return self.unpack("I", 4)

    def u64(self) -> int:
        return self.unpack("Q", 8)

    def string(self) -> str:
        n = self.u64()
        return bytes(self.take(n)).decode("utf-8", errors="replace")

    def value(self, vtype: int) -> Any:
        if vtype in _SCALARS:
            return self.unpack(*_SCALARS[vtype])
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype, count = self.u32(), self.u64()
            if etype in _SCALARS and etype != 7:
                code, size = _SCALARS[etype]
                raw = self.take(size * count)
                return list(struct.unpack(f"<{count}{code}", raw)) if count else []
            return [self.value(etype) for _ in range(count)]
        raise DracoFormatError(f"Unsupported GGUF metadata value type {vtype}.")


def tensor_nbytes(ggml_type: int, n_elements: int, name: str = "") -> int:
    if ggml_type in FLOAT_TYPES:
        return n_elements * FLOAT_TYPES[ggml_type][1]
    if ggml_type in BLOCK_TYPES:
        qk, nb = BLOCK_TYPES[ggml_type]
        if n_elements % qk:
            raise DracoFormatError(
                f"GGUF tensor '{name}' has {n_elements} elements, not a multiple of block size {qk} "
                f"for ggml type {ggml_type}."
            )
        return n_elements // qk * nb
    raise DracoFormatError(f"GGUF tensor '{name}' has unsupported ggml type {ggml_type}.")


@dataclass
class GGUFTensor:
    """Directory entry: ``info`` (shape, absolute offset, bytes) plus the
    ggml type the kernels take (Q2_K / Q3_K / Q6_K tagged with their field order)."""

    info: GgufTensorInfo
    kernel_type: int

    @property
    def name(self) -> str:
        return self.info.name

    @property
    def shape(self) -> Tuple[int, ...]:
        return self.info.shape

    @property
    def nbytes(self) -> int:
        return self.info.nbytes


class GGUFFile:
    """Opens and maps a ``.gguf`` file; ``payload(name)`` is zero-copy."""

    def __init__(self, path: str, field_order: str = "reference") -> None:
        if field_order not in ("reference", "ggml"):
            raise ValueError(f"field_order must be 'reference' or 'ggml', got {field_order!r}")
        self.path = path
        self.field_order = field_order
        self._file = open(path, "rb")
        self._map: Optional[mmap.mmap] = None
        try:
            size = os.fstat(self._file.fileno()).st_size
            if size < 24:
                raise DracoFormatError(f"'{path}' is too small to be a GGUF file ({size} bytes).")
            self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
            self.file_size = size
            view = memoryview(self._map)
            magic = bytes(view[:4])
            if magic != GGUF_MAGIC:
                raise DracoFormatError(f"Not a GGUF file: bad magic {magic!r} in '{path}'.")
            cur = _Cursor(view, 4, "header")
            self.version = cur.u32()
            if self.version not in (1, 2, 3):
                raise DracoFormatError(f"Unsupported GGUF version {self.version} in '{path}' (supported: 1-3).")
            n_tensors, n_kv = cur.u64(), cur.u64()
            cur.what = "metadata"
            meta: Dict[str, Any] = {}
            for _ in range(n_kv):
                key = cur.string()
                meta[key] = cur.value(cur.u32())
            self.metadata = meta
            align = meta.get("general.alignment", 32)
            if not isinstance(align, int) or isinstance(align, bool) or align <= 0 or align % 8:
                raise DracoFormatError(
                    f"Invalid GGUF alignment {align!r} in '{path}' (must be a positive multiple of 8)."
                )
            self.alignment = align
            cur.what = "tensor info"
            raw: List[Tuple[str, Tuple[int, ...], int, int]] = []
            for _ in range(n_tensors):
                name = cur.string()
                nd = cur.u32()
                if nd > 8:
                    raise DracoFormatError(f"GGUF tensor '{name}' has {nd} dimensions.")
                dims = tuple(cur.u64() for _ in range(nd))
                ttype, rel = cur.u32(), cur.u64()
                raw.append((name, dims, ttype, rel))
            self.data_offset = -(-cur.pos // align) * align
            self._tensors: Dict[str, GGUFTensor] = {}
            for name, dims, ttype, rel in raw:
                if name in self._tensors:
                    raise DracoFormatError(f"Duplicate GGUF tensor name '{name}'.")
                n = int(np.prod(dims, dtype=np.int64)) if dims else 1
                nbytes = tensor_nbytes(ttype, n, name)
                off = self.data_offset + rel
                if off + nbytes > size:
                    raise DracoFormatError(
                        f"GGUF tensor '{name}' extends past the end of the file ({off}+{nbytes} > {size})."
                    )
                info = GgufTensorInfo(name=name, ggml_type=ttype, shape=tuple(reversed(dims)), offset=off,
                                      nbytes=nbytes, alignment=align,
                                      dtype=FLOAT_TYPES[ttype][0] if ttype in FLOAT_TYPES else "f32")
                ktype = ttype | GGML_ORDER if (ttype in ORDER_TYPES and field_order == "ggml") else ttype
                self._tensors[name] = GGUFTensor(info, ktype)
        except Exception:
            self.close()
            raise

    # -- directory -------------------------------------------------------
    def tensor_names(self) -> List[str]:
        return list(self._tensors)

    def tensors(self) -> Iterator[GGUFTensor]:
        return iter(self._tensors.values())

    def tensor(self, name: str) -> GGUFTensor:
        if name not in self._tensors:
            raise KeyError(f"No tensor named '{name}' in '{self.path}'.")
        return self._tensors[name]

    # -- payloads --------------------------------------------------------
    def payload(self, name: str) -> np.ndarray:
        """Read-only uint8 view of the tensor's bytes in the mapping (no copy)."""
        if self._map is None:
            raise DracoFormatError(f"'{self.path}' is closed.")
        t = self.tensor(name)
        return np.frombuffer(self._map, dtype=np.uint8, count=t.nbytes, offset=t.info.offset)

    def close(self) -> None:
        if self._map is not None:
            try:
                self._map.close()
            except BufferError:
                # a payload view is still alive; the mapping goes with it
                pass
            self._map = None
        if not self._file.closed:
            self._file.close()

    def __enter__(self) -> "GGUFFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
