"""GGUF file -> HBM: packed blocks arrive byte-identical (through small
pinned chunks), float tensors keep dtype and shape, and the decode GEMV runs
on the uploaded blocks, including Q6_K blocks in upstream ggml order."""

import numpy as np
import pytest
import torch

from dracort_amd.format.gguf import Q6K_D_LAST
from dracort_amd.format.gguf_file import GGUFFile
from dracort_amd.kernels import gguf_gemv
from dracort_amd.quantization.gguf import GGUFQuantizedWeight
from dracort_amd.weights import upload_gguf
from oracle import matmul_ref
from tests.gguf_cases import Q4_K, Q6_K, Q8_0, activations, check_close, quantized
from tests.gguf_writer import q6k_to_ggml_order, write_gguf

pytestmark = pytest.mark.gpu


def _file(tmp_path, q6k_ggml: bool):
    q4k, w4 = quantized(Q4_K, 256, 512, 41)
    q6k, w6 = quantized(Q6_K, 128, 1024, 42)
    q80, w8 = quantized(Q8_0, 96, 256, 43)
    norm = np.random.default_rng(44).standard_normal(512, dtype=np.float32)
    emb = np.random.default_rng(45).standard_normal((16, 64), dtype=np.float32).astype(np.float16)
    q6_payload = q6k_to_ggml_order(q6k) if q6k_ggml else q6k
    tensors = [
        ("blk.0.ffn_gate.weight", (256, 512), Q4_K, q4k.tobytes()),
        ("blk.0.ffn_down.weight", (128, 1024), Q6_K, q6_payload.tobytes()),
        ("blk.0.attn_q.weight", (96, 256), Q8_0, q80.tobytes()),
        ("output_norm.weight", (512,), 0, norm.tobytes()),
        ("token_embd.weight", (16, 64), 1, emb.tobytes()),
    ]
    path = str(tmp_path / "m.gguf")
    write_gguf(path, [("general.architecture", "str", "llama")], tensors)
    return path, tensors, {"gate": w4, "down": w6, "q": w8}, norm, emb


@pytest.mark.parametrize("q6k_ggml", [False, True])
def test_upload_and_gemv(tmp_path, q6k_ggml):
    path, tensors, ref_w, norm, emb = _file(tmp_path, q6k_ggml)
    print(f"upload q6k_ggml={q6k_ggml}", flush=True)
    with GGUFFile(path, field_order="ggml" if q6k_ggml else "reference") as g:
        up = upload_gguf(g, chunk_bytes=4096)
        for name, shape, ttype, payload in tensors:
            t = up[name]
            data = t.data if isinstance(t, GGUFQuantizedWeight) else t
            assert data.is_cuda
            assert data.contiguous().view(torch.uint8).cpu().numpy().tobytes() == payload, name
    gate, down, q = up["blk.0.ffn_gate.weight"], up["blk.0.ffn_down.weight"], up["blk.0.attn_q.weight"]
    assert isinstance(gate, GGUFQuantizedWeight) and gate.shape == (256, 512)
    assert down.ggml_type == (Q6_K | Q6K_D_LAST if q6k_ggml else Q6_K)
    assert up["output_norm.weight"].dtype == torch.float32
    assert torch.equal(up["output_norm.weight"].cpu(), torch.from_numpy(norm))
    assert up["token_embd.weight"].dtype == torch.float16 and up["token_embd.weight"].shape == (16, 64)
    assert torch.equal(up["token_embd.weight"].cpu(), torch.from_numpy(emb))
    for wq, key in ((gate, "gate"), (down, "down"), (q, "q")):
        k = wq.shape[1]
        x = activations(1, k, 7, torch.bfloat16)
        y = gguf_gemv(x.cuda(), wq.data, wq.ggml_type, wq.shape).cpu().numpy()
        check_close(y, matmul_ref.linear_ref(x.float().numpy(), ref_w[key]), f"uploaded {key}")


def test_upload_subset_default_chunk(tmp_path):
    path, tensors, _, _, _ = _file(tmp_path, False)
    with GGUFFile(path) as g:
        up = upload_gguf(g, names=["blk.0.attn_q.weight"])
    assert list(up) == ["blk.0.attn_q.weight"]
    assert up["blk.0.attn_q.weight"].data.cpu().numpy().tobytes() == tensors[2][3]
