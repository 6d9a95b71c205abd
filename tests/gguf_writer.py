"""A small GGUF writer for building test files (metadata of every value type,
2-D quantized tensors and float vectors), written from the container format
the reader documents; no part of the reference is used."""

from __future__ import annotations

import struct
from typing import Any, Dict, List, Sequence, Tuple

import numpy as np

_SCALAR = {"u8": (0, "B"), "i8": (1, "b"), "u16": (2, "H"), "i16": (3, "h"), "u32": (4, "I"), "i32": (5, "i"),
           "f32": (6, "f"), "bool": (7, "?"), "u64": (10, "Q"), "i64": (11, "q"), "f64": (12, "d")}


def _s(text: str) -> bytes:
    b = text.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(kind: str, v: Any) -> bytes:
    if kind == "str":
        return struct.pack("<I", 8) + _s(v)
    if kind.startswith("arr:"):
        ek = kind[4:]
        out = struct.pack("<IIQ", 9, 8 if ek == "str" else _SCALAR[ek][0], len(v))
        for e in v:
            out += _s(e) if ek == "str" else struct.pack("<" + _SCALAR[ek][1], e)
        return out
    t, code = _SCALAR[kind]
    return struct.pack("<I", t) + struct.pack("<" + code, v)


def write_gguf(path: str, metadata: Sequence[Tuple[str, str, Any]],
               tensors: Sequence[Tuple[str, Tuple[int, ...], int, bytes]],
               version: int = 3, alignment: int = 32, magic: bytes = b"GGUF") -> List[int]:
    """tensors: (name, numpy shape, ggml type, payload).  Returns each
    tensor's offset relative to the data section."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    meta = b"".join(_s(k) + _value(kind, v) for k, kind, v in metadata)
    infos, rel, offs = b"", 0, []
    for name, shape, ttype, payload in tensors:
        dims = tuple(reversed(shape))
        infos += _s(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        infos += struct.pack("<IQ", ttype, rel)
        offs.append(rel)
        rel += len(payload)
        rel = -(-rel // alignment) * alignment
    body = head + meta + infos
    pad = (-len(body)) % alignment
    data = b""
    for (name, shape, ttype, payload), off in zip(tensors, offs):
        data += b"\0" * (off - len(data)) + payload
    with open(path, "wb") as f:
        f.write(body + b"\0" * pad + data)
    return offs


def q6k_to_ggml_order(blocks: np.ndarray) -> np.ndarray:
    """Reference-order Q6_K blocks (d first) -> upstream ggml order (d last)."""
    b = blocks.reshape(-1, 210)
    return np.concatenate([b[:, 2:], b[:, :2]], axis=1).reshape(-1)
