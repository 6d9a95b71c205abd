"""GGUF container reader (host side): metadata of every value type, tensor
directory (reversed dims, aligned data section, absolute offsets), zero-copy
payloads, the Q2_K / Q3_K / Q6_K field-order tag, and the reference's rejection cases
(bad magic / version / alignment, tensors past the end, partial blocks)."""

import os

import numpy as np
import pytest
import torch

from dracort_amd.exceptions import DracoFormatError
from dracort_amd.format.gguf import Q6K_D_LAST
from dracort_amd.format.gguf_file import GGUFFile
from dracort_amd.quantization import quantize
from tests.gguf_writer import write_gguf

META = [
    ("general.architecture", "str", "llama"),
    ("general.name", "str", "tiny"),
    ("llama.block_count", "u32", 2),
    ("llama.embedding_length", "u64", 256),
    ("llama.rope.freq_base", "f32", 500000.0),
    ("x.u8", "u8", 200), ("x.i8", "i8", -5), ("x.u16", "u16", 60000), ("x.i16", "i16", -30000),
    ("x.i32", "i32", -7), ("x.i64", "i64", -(1 << 40)), ("x.f64", "f64", 0.125), ("x.bool", "bool", True),
    ("tokenizer.ggml.tokens", "arr:str", ["<s>", "</s>", "hello", "wörld"]),
    ("tokenizer.ggml.token_type", "arr:i32", [3, 3, 1, 1]),
    ("x.flags", "arr:bool", [True, False, True]),
]


def _tensors():
    rng = np.random.default_rng(0)
    w = torch.from_numpy(rng.standard_normal((8, 512), dtype=np.float32) * np.float32(0.02))
    q4k = quantize(w, 12).numpy().tobytes()
    q6k = quantize(w[:4], 14).numpy().tobytes()
    q80 = quantize(w[:3, :64], 8).numpy().tobytes()
    q3k = quantize(w[:2], 11).numpy().tobytes()
    q51 = quantize(w[:5, :96], 7).numpy().tobytes()
    norm = rng.standard_normal(256, dtype=np.float32)
    return [
        ("blk.0.ffn_gate.weight", (8, 512), 12, q4k),
        ("blk.0.ffn_down.weight", (4, 512), 14, q6k),
        ("blk.0.attn_q.weight", (3, 64), 8, q80),
        ("blk.0.attn_k.weight", (2, 512), 11, q3k),
        ("blk.0.attn_v.weight", (5, 96), 7, q51),
        ("output_norm.weight", (256,), 0, norm.tobytes()),
    ], norm


def test_roundtrip_metadata_and_directory(tmp_path):
    path = str(tmp_path / "t.gguf")
    tensors, norm = _tensors()
    rel = write_gguf(path, META, tensors)
    with GGUFFile(path) as g:
        assert g.version == 3 and g.alignment == 32
        for k, kind, v in META:
            got = g.metadata[k]
            if kind == "f32":
                assert got == pytest.approx(v)
            else:
                assert got == v, k
        assert g.data_offset % 32 == 0
        assert g.tensor_names() == [t[0] for t in tensors]
        for (name, shape, ttype, payload), r in zip(tensors, rel):
            t = g.tensor(name)
            assert t.shape == shape and t.info.ggml_type == ttype and t.nbytes == len(payload)
            assert t.info.offset == g.data_offset + r and t.info.offset % 32 == 0
            p = g.payload(name)
            assert p.tobytes() == payload
            assert not p.flags.writeable and not p.flags.owndata  # a view of the mapping
            del p
        assert g.tensor("output_norm.weight").info.dtype == "f32"
        assert g.tensor("blk.0.ffn_down.weight").kernel_type == 14
        with pytest.raises(KeyError):
            g.tensor("nope")
    with GGUFFile(path, field_order="ggml") as g:
        assert g.tensor("blk.0.ffn_down.weight").kernel_type == 14 | Q6K_D_LAST
        assert g.tensor("blk.0.attn_k.weight").kernel_type == 11 | Q6K_D_LAST
        assert g.tensor("blk.0.ffn_gate.weight").kernel_type == 12
        assert g.tensor("blk.0.attn_v.weight").kernel_type == 7


def test_custom_alignment(tmp_path):
    path = str(tmp_path / "a.gguf")
    tensors, _ = _tensors()
    write_gguf(path, META + [("general.alignment", "u32", 64)], tensors, alignment=64)
    with GGUFFile(path) as g:
        assert g.alignment == 64 and g.data_offset % 64 == 0
        for name, _, _, payload in tensors:
            assert g.tensor(name).info.offset % 64 == 0
            assert g.payload(name).tobytes() == payload


@pytest.mark.parametrize("case", ["magic", "version", "alignment", "past_end", "partial_block", "tiny", "dup"])
def test_rejections(tmp_path, case):
    path = str(tmp_path / f"{case}.gguf")
    tensors, _ = _tensors()
    if case == "magic":
        write_gguf(path, META, tensors, magic=b"GGUG")
    elif case == "version":
        write_gguf(path, META, tensors, version=4)
    elif case == "alignment":
        write_gguf(path, META + [("general.alignment", "u32", 12)], tensors)
    elif case == "past_end":
        write_gguf(path, META, tensors)
        with open(path, "r+b") as f:
            f.truncate(os.path.getsize(path) - 100)
    elif case == "partial_block":
        write_gguf(path, META, [("w", (2, 100), 12, b"\0" * 144)])
    elif case == "tiny":
        with open(path, "wb") as f:
            f.write(b"GGUF\3\0\0\0")
    elif case == "dup":
        write_gguf(path, META, [tensors[0], tensors[0]])
    with pytest.raises(DracoFormatError):
        GGUFFile(path)


def test_truncated_metadata(tmp_path):
    path = str(tmp_path / "m.gguf")
    write_gguf(path, META, [])
    size = os.path.getsize(path)
    with open(path, "r+b") as f:
        f.truncate(size - 40)
    with pytest.raises(DracoFormatError):
        GGUFFile(path)
