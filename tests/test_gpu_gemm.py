"""GPU parity: prefill GEMM (weight tiles decoded into LDS, bf16 MFMA, fp32
accumulate) against the oracle's fp64 dequant-then-matmul, <= 1e-3."""

import numpy as np
import pytest
import torch

from dracort_amd import _native
from dracort_amd.kernels import gemm_workspace_bytes, gguf_gemm, gguf_linear
from oracle import matmul_ref
from tests.gguf_cases import NAMES, Q4_K, Q6_K, Q8_0, TYPES, activations, check_close, quantized

pytestmark = pytest.mark.gpu


def _run(qtype, n, k, m, seed=0, bias=None):
    blocks, w = quantized(qtype, n, k, seed)
    x = activations(m, k, seed, torch.bfloat16)
    ref = matmul_ref.linear_ref(x.float().numpy(), w)
    y = gguf_gemm(x.cuda(), torch.from_numpy(blocks).cuda(), qtype, (n, k), bias=bias).cpu().numpy()
    return y, ref


@pytest.mark.parametrize("qtype", TYPES)
def test_gemm_tile_edges(qtype):
    qk = 256 if qtype in (Q4_K, Q6_K) else 32
    for n, k, m in ((1, qk, 1), (130, 2 * qk, 129), (257, 3 * qk, 17), (64, 8 * qk, 300)):
        print(f"gemm {NAMES[qtype]} [{n},{k}] m={m}", flush=True)
        y, ref = _run(qtype, n, k, m, seed=n + m)
        check_close(y, ref, f"gemm {NAMES[qtype]} [{n},{k}] m={m}")


@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
def test_gemm_prefill_q4k_full_shape(n, k):
    print(f"gemm Q4_K [{n},{k}] m=512", flush=True)
    y, ref = _run(Q4_K, n, k, 512, seed=1)
    check_close(y, ref, f"gemm Q4_K [{n},{k}] m=512")


def test_gemm_via_linear_dispatch_and_bias():
    blocks, w = quantized(Q6_K, 512, 1024, 4)
    x = activations(40, 1024, 4, torch.bfloat16)
    b = torch.from_numpy(np.random.default_rng(4).standard_normal(512, dtype=np.float32))
    y = gguf_linear(x.cuda(), torch.from_numpy(blocks).cuda(), Q6_K, (512, 1024), bias=b.cuda()).cpu().numpy()
    ref = matmul_ref.linear_ref(x.float().numpy(), w) + b.numpy()
    check_close(y, ref, "linear bf16 m=40")


def test_gemm_q8_0_k_not_multiple_of_64():
    y, ref = _run(Q8_0, 96, 96, 70, seed=8)
    check_close(y, ref, "gemm Q8_0 K=96")


def test_gemm_q4k_large_activations_row_scaling():
    """Rows whose largest |x| is beyond float16's range are scaled by a power
    of two for the float16 matrix cores and unscaled on the output."""
    blocks, w = quantized(Q4_K, 256, 1024, 11)
    x = activations(70, 1024, 11, torch.float32)
    x[3, 5] = 1.5e5
    x[17, 900] = -7.0e6
    x[40] *= 3.0e4  # a whole row far beyond 65504
    x = x.to(torch.bfloat16)
    print("gemm Q4_K large activations", flush=True)
    y = gguf_gemm(x.cuda(), torch.from_numpy(blocks).cuda(), Q4_K, (256, 1024)).cpu().numpy()
    ref = matmul_ref.linear_ref(x.float().numpy(), w)
    for r in (3, 17, 40, 0, 69):
        check_close(y[r], ref[r], f"gemm Q4_K large x row {r}")


def test_gemm_q4k_without_workspace_matches():
    """A NULL workspace runs the workspace-free kernel; both agree with the oracle."""
    n, k, m = 384, 1024, 200
    blocks, w = quantized(Q4_K, n, k, 12)
    x = activations(m, k, 12, torch.bfloat16).cuda()
    wq = torch.from_numpy(blocks).cuda()
    y0 = torch.empty((m, n), dtype=torch.float32, device="cuda")
    lib = _native.load()
    print("gemm Q4_K workspace-free", flush=True)
    rc = lib.draco_gguf_gemm(Q4_K, wq.data_ptr(), wq.numel(), x.data_ptr(), None, y0.data_ptr(), m, n, k, None, 0,
                             torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _native.last_error()
    y1 = gguf_gemm(x, wq, Q4_K, (n, k))
    ref = matmul_ref.linear_ref(x.cpu().float().numpy(), w)
    check_close(y0.cpu().numpy(), ref, "gemm Q4_K no workspace")
    check_close(y1.cpu().numpy(), ref, "gemm Q4_K workspace")
    assert gemm_workspace_bytes(Q4_K, m, k) > 0


def _q4k_ws_required(m, k):
    al = lambda v: (v + 255) // 256 * 256  # noqa: E731
    return al(m * k * 2) + al(3 * m * (k // 32) * 2) + al(m * 4)


@pytest.mark.parametrize("n,k,m", [(1000, 4096, 200), (4096, 14336, 64)])
def test_gemm_q4k_split_k(n, k, m):
    """Few output tiles: the workspace's split-K room splits the K range over
    several workgroups per tile, and a second launch adds their partial sums in
    split order (bit-identical from run to run); a workspace without the room
    runs unsplit.  Both agree with the oracle."""
    blocks, w = quantized(Q4_K, n, k, 21)
    x = activations(m, k, 21, torch.bfloat16).cuda()
    wq = torch.from_numpy(blocks).cuda()
    b = torch.from_numpy(np.random.default_rng(21).standard_normal(n, dtype=np.float32)).cuda()
    full = gemm_workspace_bytes(Q4_K, m, k)
    assert full > _q4k_ws_required(m, k)
    print(f"gemm Q4_K split-K [{n},{k}] m={m}", flush=True)
    ws = torch.empty(full, dtype=torch.uint8, device="cuda")
    y1 = gguf_gemm(x, wq, Q4_K, (n, k), bias=b, workspace=ws).cpu()
    y2 = gguf_gemm(x, wq, Q4_K, (n, k), bias=b, workspace=ws).cpu()
    assert torch.equal(y1, y2)
    ws_min = torch.empty(_q4k_ws_required(m, k), dtype=torch.uint8, device="cuda")
    y3 = gguf_gemm(x, wq, Q4_K, (n, k), bias=b, workspace=ws_min).cpu()
    ref = matmul_ref.linear_ref(x.cpu().float().numpy(), w) + b.cpu().numpy()
    check_close(y1.numpy(), ref, f"gemm Q4_K split-K [{n},{k}] m={m}")
    check_close(y3.numpy(), ref, f"gemm Q4_K unsplit [{n},{k}] m={m}")


def test_gemm_q4k_tail_split():
    """A grid of whole rounds plus a partial one (2048 x 5120: 320 tiles of
    256 x 128 on 256 CUs): the partial round's tiles run in parts of K whose
    raw sums a second launch adds in split order for their columns only, the
    rest of the tiles whole.  Deterministic from run to run and, like the
    unsplit launch (workspace without the split room), within the bar of the
    oracle."""
    m, n, k = 2048, 5120, 1024
    blocks, w = quantized(Q4_K, n, k, 31)
    x = activations(m, k, 31, torch.bfloat16).cuda()
    wq = torch.from_numpy(blocks).cuda()
    b = torch.from_numpy(np.random.default_rng(31).standard_normal(n, dtype=np.float32)).cuda()
    print(f"gemm Q4_K tail split [{n},{k}] m={m}", flush=True)
    ws = torch.empty(gemm_workspace_bytes(Q4_K, m, k), dtype=torch.uint8, device="cuda")
    y1 = gguf_gemm(x, wq, Q4_K, (n, k), bias=b, workspace=ws).cpu()
    y2 = gguf_gemm(x, wq, Q4_K, (n, k), bias=b, workspace=ws).cpu()
    assert torch.equal(y1, y2)
    ws_min = torch.empty(_q4k_ws_required(m, k), dtype=torch.uint8, device="cuda")
    y3 = gguf_gemm(x, wq, Q4_K, (n, k), bias=b, workspace=ws_min).cpu()
    ref = matmul_ref.linear_ref(x.cpu().float().numpy(), w) + b.cpu().numpy()
    check_close(y1.numpy(), ref, f"gemm Q4_K tail split [{n},{k}] m={m}")
    check_close(y3.numpy(), ref, f"gemm Q4_K unsplit [{n},{k}] m={m}")
    # the whole tiles' columns are the unsplit launch's bits
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    full = (8 * 40 // cus) * cus  # whole rounds of the 8 x 40 tiles
    nt = full // 8 * 128
    assert torch.equal(y1[:, :nt], y3[:, :nt])


def test_gemm_q4k_m2048_bias_via_linear():
    blocks, w = quantized(Q4_K, 1024, 2048, 13)
    x = activations(2048, 2048, 13, torch.bfloat16)
    b = torch.from_numpy(np.random.default_rng(13).standard_normal(1024, dtype=np.float32))
    print("linear Q4_K m=2048 bias", flush=True)
    y = gguf_linear(x.cuda(), torch.from_numpy(blocks).cuda(), Q4_K, (1024, 2048), bias=b.cuda()).cpu().numpy()
    ref = matmul_ref.linear_ref(x.float().numpy(), w) + b.numpy()
    check_close(y, ref, "linear Q4_K m=2048")


def test_gemm_q4k_small_magnitude_rows_via_linear():
    """Every row is normalised by a power of two into float16's normal range,
    so rows of tiny values keep full precision: rows at 1e-2 .. 1e-9 scale, one
    row mixing magnitudes from 1e-9 to 1e3, a zero row and a row of bf16
    subnormals, through gguf_linear (the workspace GEMM) at M > 16.  Each row is
    held on its own to the 1e-3 bar against the fp64 oracle."""
    n, k, m = 512, 1024, 40
    blocks, w = quantized(Q4_K, n, k, 21)
    x = activations(m, k, 21, torch.float32)
    scales = {0: 1e-2, 1: 1e-4, 2: 1e-6, 3: 1e-9, 4: 1e-20, 5: 1e-30}
    for r, sc in scales.items():
        x[r] *= sc
    x[6] *= torch.logspace(-9, 3, k)  # mixed magnitudes within one row
    x[7] = 0.0
    x[8] = torch.from_numpy(np.full(k, 2.0 ** -130, dtype=np.float32)) * torch.sign(x[8])  # bf16 subnormals
    x = x.to(torch.bfloat16)
    print("linear Q4_K small-magnitude rows m=40", flush=True)
    y = gguf_linear(x.cuda(), torch.from_numpy(blocks).cuda(), Q4_K, (n, k)).cpu().numpy()
    ref = matmul_ref.linear_ref(x.float().numpy(), w)
    assert np.all(y[7] == 0.0), "zero row must give exact zeros"
    for r in list(scales) + [6, 8, 9, 39]:
        check_close(y[r], ref[r], f"linear Q4_K row {r}")
