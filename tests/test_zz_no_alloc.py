"""draco_gguf_linear_noalloc: the prefill GEMM whose workspace is the
library's static per-GPU scratch array, called through the C ABI and checked
against draco_gguf_linear (caller-provided workspace) and the fp64 oracle, on
two calls in a row, the second one smaller."""

import ctypes

import numpy as np
import pytest
import torch

from dracort_amd import _native
from dracort_amd.kernels import gguf_linear
from oracle import matmul_ref
from tests.gguf_cases import Q4_K, Q6_K, activations, check_close, quantized

BF16 = _native.DRACO_DTYPE_BF16
FAKE = 0x10000  # aligned, never dereferenced: the call below fails validation first


def _noalloc(wq, qtype, x, y, m, n, k, bias=None):
    lib = _native.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.draco_gguf_linear_noalloc(qtype, wq.data_ptr(), wq.numel(), x.data_ptr(), BF16,
                                         bias.data_ptr() if bias is not None else None, y.data_ptr(), m, n, k, stream)


@pytest.mark.gpu
def test_linear_noalloc_matches_linear_on_two_calls():
    """The first call is the process's first use of the scratch (its address is
    looked up then); the second, smaller call reuses what the first left."""
    cases = [(Q4_K, 512, 2048, 300, 1, True), (Q4_K, 256, 1024, 40, 2, False)]
    for qtype, n, k, m, seed, with_bias in cases:
        print(f"linear_noalloc type {qtype} [{n},{k}] m={m}", flush=True)
        blocks, w = quantized(qtype, n, k, seed)
        x = activations(m, k, seed, torch.bfloat16).cuda()
        wq = torch.from_numpy(blocks).cuda()
        bias = torch.from_numpy(np.random.default_rng(seed).standard_normal(n).astype(np.float32)).cuda() \
            if with_bias else None
        y1 = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        rc = _noalloc(wq, qtype, x, y1, m, n, k, bias)
        assert rc == 0, _native.last_error()
        y0 = gguf_linear(x, wq, qtype, (n, k), bias=bias)  # the existing entry point, its own workspace
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), "noalloc and workspace GEMMs must give the same bits"
        ref = matmul_ref.linear_ref(x.cpu().float().numpy(), w)
        if bias is not None:
            ref = ref + bias.cpu().numpy()
        check_close(y1.cpu().numpy(), ref, f"linear_noalloc [{n},{k}] m={m}")


@pytest.mark.gpu
def test_linear_noalloc_types_without_scratch_and_small_m():
    """Q6_K (its GEMM needs no workspace) and m <= 16 (the GEMV) pass straight through."""
    for qtype, m in ((Q6_K, 33), (Q4_K, 7)):
        n, k = 256, 512
        blocks, w = quantized(qtype, n, k, 5)
        x = activations(m, k, 5, torch.bfloat16).cuda()
        wq = torch.from_numpy(blocks).cuda()
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        assert _noalloc(wq, qtype, x, y, m, n, k) == 0, _native.last_error()
        check_close(y.cpu().numpy(), matmul_ref.linear_ref(x.cpu().float().numpy(), w), f"noalloc {qtype} m={m}")


def test_linear_noalloc_rejects_work_beyond_the_scratch():
    """4096 rows of 14336 need ~128 MB of workspace: refused before any launch."""
    lib = _native.load()
    need = lib.draco_gguf_gemm_workspace_size(Q4_K, 4096, 14336)
    assert need > _native.DRACO_GGUF_NOALLOC_SCRATCH_BYTES
    rc = lib.draco_gguf_linear_noalloc(Q4_K, FAKE, 1 << 40, FAKE, BF16, None, FAKE, 4096, 4096, 14336, None)
    assert rc == _native.DRACO_EWORKSPACE
    assert "maximum" in _native.last_error()
    # the workspace the GEMM requires at 2048 x 14336 fits (the optional split-K room does not)
    al = lambda v: (v + 255) // 256 * 256  # noqa: E731
    m, k = 2048, 14336
    assert al(m * k * 2) + al(3 * m * (k // 32) * 2) + al(m * 4) <= _native.DRACO_GGUF_NOALLOC_SCRATCH_BYTES
