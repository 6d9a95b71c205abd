"""Executor GPU tier: ``_linear`` on a GGUF file's tensors through HBM-resident
packed blocks (numpy in/out like the reference's CPU tier, or device tensors),
with a float32 bias from the file, against the oracle's fp64 closed form."""

import numpy as np
import pytest
import torch

from dracort_amd.format.gguf_file import GGUFFile
from dracort_amd.runtime import GGUFGpuKernel
from oracle import matmul_ref
from tests.gguf_cases import Q4_K, Q6_K, activations, check_close, quantized
from tests.gguf_writer import write_gguf

pytestmark = pytest.mark.gpu


def _model(tmp_path):
    q4k, w4 = quantized(Q4_K, 512, 1024, 51)
    q6k, w6 = quantized(Q6_K, 256, 512, 52)
    bias = np.random.default_rng(53).standard_normal(512, dtype=np.float32)
    path = str(tmp_path / "tier.gguf")
    write_gguf(path, [("general.architecture", "str", "llama")], [
        ("blk.0.ffn_up.weight", (512, 1024), Q4_K, q4k.tobytes()),
        ("blk.0.ffn_up.bias", (512,), 0, bias.tobytes()),
        ("blk.0.attn_k.weight", (256, 512), Q6_K, q6k.tobytes()),
    ])
    return path, w4, w6, bias


def test_linear_numpy_and_device(tmp_path):
    path, w4, w6, bias = _model(tmp_path)
    tier = GGUFGpuKernel()
    with GGUFFile(path) as g:
        for m in (1, 5, 40):
            x = activations(m, 1024, m, torch.float32).numpy()
            print(f"tier linear numpy m={m}", flush=True)
            y = tier.linear(g, "blk.0.ffn_up.weight", x, bias_name="blk.0.ffn_up.bias")
            assert isinstance(y, np.ndarray) and y.shape == (m, 512)
            check_close(y, matmul_ref.linear_ref(x, w4) + bias, f"tier numpy m={m}")
        resident = tier.resident_bytes()
        xb = activations(64, 512, 9, torch.bfloat16)
        print("tier linear device bf16 m=64", flush=True)
        yd = tier.linear(g, "blk.0.attn_k.weight", xb.cuda())
        assert yd.is_cuda and yd.shape == (64, 256)
        check_close(yd.cpu().numpy(), matmul_ref.linear_ref(xb.float().numpy(), w6), "tier device m=64")
        assert tier.resident_bytes() > resident
        # cached: a second call uploads nothing more
        before = tier.resident_bytes()
        tier.linear(g, "blk.0.attn_k.weight", xb.cuda())
        assert tier.resident_bytes() == before


def test_matmul_reference_signature(tmp_path):
    path, w4, _, _ = _model(tmp_path)
    tier = GGUFGpuKernel()
    with GGUFFile(path) as g:
        t = g.tensor("blk.0.ffn_up.weight")
        x = activations(3, 1024, 3, torch.float32).numpy()
        print("tier matmul", flush=True)
        y = tier.matmul(x, t.info, g.payload("blk.0.ffn_up.weight").tobytes())
    check_close(y, matmul_ref.linear_ref(x, w4), "tier matmul")
