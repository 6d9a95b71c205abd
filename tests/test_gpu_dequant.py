"""GPU parity: bit-exact dequantization against the reference's golden vectors
and the oracle, through the C ABI (via dracort_amd.kernels)."""

import os

import numpy as np
import pytest
import torch

from dracort_amd.exceptions import DracoFormatError
from dracort_amd.kernels import gguf_dequantize
from oracle import gguf_ref
from tests.gguf_cases import NAMES, Q4_0, Q4_K, Q6_K, Q8_0, TYPES, quantized

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _dev_bytes(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).reshape(-1)).cuda()


@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_matches_reference_golden(qtype):
    z = np.load(os.path.join(GOLDEN, "gguf_dequant_golden.npz"))
    name = NAMES[qtype]
    blocks = z[f"{name}_blocks"]
    qk = gguf_ref.BLOCK_LAYOUT[qtype][0]
    nb = blocks.shape[0]
    expect = z[f"{name}_expect_bits"]
    print(f"dequant golden {name} nb={nb}", flush=True)
    # as one row and as rows of one block (odd row byte offsets for the 2-byte-aligned types)
    for n, k in ((1, nb * qk), (nb, qk)):
        got = gguf_dequantize(_dev_bytes(blocks), qtype, (n, k)).cpu().numpy()
        assert np.array_equal(got.reshape(-1).view(np.uint32), expect), (name, n, k)
    if qtype == Q6_K:
        up = gguf_ref.q6k_reorder(blocks, to_upstream=True)
        got = gguf_dequantize(_dev_bytes(up), Q6_K | 0x100, (nb, qk)).cpu().numpy()
        assert np.array_equal(got.reshape(-1).view(np.uint32), expect)


SHAPES = {
    Q8_0: [(4096, 4096), (3, 96), (1, 32)],
    Q4_0: [(1024, 4096), (14336, 4096), (5, 96), (1, 32)],
    Q4_K: [(14336, 4096), (4096, 14336), (3, 256), (1, 512)],
    Q6_K: [(4096, 14336), (8192, 4096), (3, 256), (2, 768)],
}


@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_bit_exact_at_config_shapes(qtype):
    for n, k in SHAPES[qtype]:
        print(f"dequant {NAMES[qtype]} [{n}, {k}]", flush=True)
        blocks, ref = quantized(qtype, n, k, seed=n + k)
        got = gguf_dequantize(_dev_bytes(blocks), qtype, (n, k)).cpu().numpy()
        assert got.shape == (n, k)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (NAMES[qtype], n, k)


def test_dequant_q6k_upstream_layout_at_shape():
    blocks, ref = quantized(Q6_K | 0x100, 64, 4096, seed=3)
    got = gguf_dequantize(_dev_bytes(blocks), Q6_K | 0x100, (64, 4096)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_rejects_truncated_payload_on_gpu():
    blocks, _ = quantized(Q4_K, 4, 256, seed=1)
    with pytest.raises(DracoFormatError):
        gguf_dequantize(_dev_bytes(blocks[:-16]), Q4_K, (4, 256))
