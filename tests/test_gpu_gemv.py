"""GPU parity: fused dequant-GEMV (decode, M = 1..16) against the oracle's
fp64 dequant-then-matmul, max elementwise relative error <= 1e-3."""

import numpy as np
import pytest
import torch

from dracort_amd.kernels import gguf_gemv, gguf_linear
from oracle import matmul_ref
from tests.gguf_cases import NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, TYPES, activations, check_close, quantized

pytestmark = pytest.mark.gpu

# Llama-3-8B projection shapes [N, K]: q/o, k/v, gate/up, down
LLAMA = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


def _run(qtype, n, k, m, xdtype, seed=0, bias=False):
    blocks, w = quantized(qtype, n, k, seed)
    x = activations(m, k, seed, xdtype)
    ref = matmul_ref.linear_ref(x.float().numpy(), w)
    b = None
    if bias:
        b = torch.from_numpy(np.random.default_rng(seed).standard_normal(n, dtype=np.float32))
        ref = ref + b.numpy().astype(np.float64)
        b = b.cuda()
    q = torch.from_numpy(blocks).cuda()
    y = gguf_gemv(x.cuda(), q, qtype, (n, k), bias=b).cpu().numpy()
    return y, ref


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
def test_gemv_llama_shapes(qtype, xdtype):
    for n, k in LLAMA:
        for m in (1, 4, 8, 16):
            print(f"gemv {NAMES[qtype]} [{n},{k}] m={m} {xdtype}", flush=True)
            y, ref = _run(qtype, n, k, m, xdtype)
            check_close(y, ref, f"{NAMES[qtype]} [{n},{k}] m={m} {xdtype}")


@pytest.mark.parametrize("qtype", TYPES)
def test_gemv_every_m_and_ragged_shapes(qtype):
    qk = 256 if qtype in (Q4_K, Q6_K) else 32
    for n, k in ((1, qk), (7, 3 * qk), (33, 5 * qk), (130, 2 * qk)):
        for m in range(1, 17):
            xd = torch.bfloat16 if m % 2 else torch.float32
            print(f"gemv {NAMES[qtype]} [{n},{k}] m={m}", flush=True)
            y, ref = _run(qtype, n, k, m, xd, seed=n * 31 + m)
            check_close(y, ref, f"{NAMES[qtype]} [{n},{k}] m={m}")


def test_gemv_bias_and_q6k_upstream_layout():
    y, ref = _run(Q4_K, 512, 1024, 3, torch.float32, seed=5, bias=True)
    check_close(y, ref, "bias")
    y, ref = _run(Q6_K | 0x100, 300, 2048, 2, torch.bfloat16, seed=6)
    check_close(y, ref, "q6k d-last")
    # the matrix-core path (16-row tiles, 8..16 activation rows) in both field orders
    for qt in (Q6_K, Q6_K | 0x100):
        for m in (8, 13, 16):
            y, ref = _run(qt, 512, 2048, m, torch.bfloat16, seed=7 + m)
            check_close(y, ref, f"q6k {qt} mfma m={m}")


def test_linear_dispatch_large_m_float32():
    """M > 16 with float32 activations runs as 16-row GEMV tiles."""
    blocks, w = quantized(Q8_0, 256, 512, 9)
    x = activations(37, 512, 9, torch.float32)
    y = gguf_linear(x.cuda(), torch.from_numpy(blocks).cuda(), Q8_0, (256, 512)).cpu().numpy()
    check_close(y, matmul_ref.linear_ref(x.numpy(), w), "linear f32 m=37")
    # an odd N (a 32001-entry vocabulary, say): every 16-row tile's output stays 16-byte aligned
    blocks, w = quantized(Q4_K, 1001, 512, 10)
    x = activations(40, 512, 10, torch.float32)
    y = gguf_linear(x.cuda(), torch.from_numpy(blocks).cuda(), Q4_K, (1001, 512)).cpu().numpy()
    check_close(y, matmul_ref.linear_ref(x.numpy(), w), "linear f32 m=40 n=1001")


def test_gemv_batched_decode_equals_sequential():
    """Rows of a batched GEMV equal single-row GEMVs (the reference's
    batched-decode == sequential-decode property, tests/runtime_cpu/
    test_batching_and_speculative.py:55-80)."""
    blocks, _ = quantized(Q4_K, 1024, 4096, 2)
    q = torch.from_numpy(blocks).cuda()
    x = activations(8, 4096, 2, torch.bfloat16).cuda()
    yb = gguf_gemv(x, q, Q4_K, (1024, 4096))
    for i in range(8):
        yi = gguf_gemv(x[i:i + 1].contiguous(), q, Q4_K, (1024, 4096))
        assert torch.allclose(yb[i], yi[0], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q6_K | 0x100])
def test_gemv_single_token_multi_step_rows(qtype):
    """One bf16 token over rows of 2, 3 and 4 steps of 64 units (K = 8192,
    11008, 14336, 16384) and row counts that leave waves empty or partly
    filled: the persistent multi-step form, plain and residual modes."""
    from dracort_amd.kernels import gguf_gemv_residual
    for n, k in ((300, 8192), (77, 11008), (4096, 14336), (5, 16384)):
        print(f"gemv x1s {qtype:#x} [{n},{k}]", flush=True)
        y, ref = _run(qtype, n, k, 1, torch.bfloat16, seed=n + k)
        check_close(y, ref, f"{qtype:#x} [{n},{k}]")
    blocks, w = quantized(qtype, 640, 11008, 3)
    x = activations(1, 11008, 3, torch.bfloat16)
    resid = torch.from_numpy(np.random.default_rng(3).standard_normal((1, 640)).astype(np.float32))
    ref = resid.numpy().astype(np.float64) + matmul_ref.linear_ref(x.float().numpy(), w)
    r = resid.cuda()
    gguf_gemv_residual(x.cuda(), torch.from_numpy(blocks).cuda(), qtype, (640, 11008), r)
    check_close(r.cpu().numpy(), ref, f"{qtype:#x} residual")


def _bf16_round(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m", [2, 4, 8])
def test_gemv_k_windows(qtype, m):
    """Float32 activation rows longer than the LDS activation image (m x k
    floats > 64 KB): the K-quant launches run as K windows of whole
    2048-column steps -- bias added by the first window, later windows through
    the residual epilogue, the bf16 copy written by the last.  Eight rows are
    windowed only when two windows cover K; Q6_K (like Q2_K / Q3_K) is not
    windowed, and Q4_0 / Q8_0 run on the float32 matrix-core kernel: both
    check the same entry points on their own paths."""
    from dracort_amd.kernels import gguf_gemv_multi, gguf_gemv_residual

    n, k = 1000, (14336 if m <= 4 else 4096)
    print(f"k windows {NAMES[qtype]} m={m}", flush=True)
    y, ref = _run(qtype, n, k, m, torch.float32, seed=80 + m, bias=True)
    check_close(y, ref, f"windows bias {NAMES[qtype]} m={m}")

    blocks, w = quantized(qtype, n, k, 90 + m)
    q = torch.from_numpy(blocks).cuda()
    x = activations(m, k, 90 + m, torch.float32)
    ref = matmul_ref.linear_ref(x.numpy(), w)
    yo = torch.full((m, n), float("nan"), device="cuda")
    yb = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
    gguf_gemv_multi(x.cuda(), [(q, n)], qtype, k, [yo], [yb])
    got = yo.cpu().numpy()
    check_close(got, ref, f"windows multi {NAMES[qtype]} m={m}")
    assert np.array_equal(yb.float().cpu().numpy(), _bf16_round(got))

    r0 = np.random.default_rng(95 + m).standard_normal((m, n), dtype=np.float32)
    resid = torch.from_numpy(r0.copy()).cuda()
    rb = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
    gguf_gemv_residual(x.cuda(), q, qtype, (n, k), resid, rb)
    got = resid.cpu().numpy()
    check_close(got, r0.astype(np.float64) + ref, f"windows residual {NAMES[qtype]} m={m}")
    assert np.array_equal(rb.float().cpu().numpy(), _bf16_round(got))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q4_0])
@pytest.mark.parametrize("m,xdtype", [(16, torch.bfloat16), (8, torch.bfloat16), (12, torch.float32)])
def test_gemv_residual_split_k(qtype, m, xdtype):
    """Long rows (K = 14336) at 8..16 activation rows with a workspace: K is
    split over several workgroups per 16-row tile and the partial sums are
    added in split order by a second launch -- the same result on every call,
    within the bar of the oracle like the unsplit launch (no workspace, or a
    workspace one byte short)."""
    from dracort_amd.kernels import gemv_residual_workspace_bytes, gguf_gemv_residual

    n, k = 512, 14336
    need = gemv_residual_workspace_bytes(qtype, m, n, k)
    assert need == 7 * m * n * 4  # 56 chunks of 256 in 7 splits of 8
    assert gemv_residual_workspace_bytes(qtype, 4, n, k) == 0  # below 8 rows: no split
    blocks, w = quantized(qtype, n, k, 120 + m)
    q = torch.from_numpy(blocks).cuda()
    x = activations(m, k, 120 + m, xdtype).cuda()
    ref = matmul_ref.linear_ref(x.cpu().float().numpy(), w)
    r0 = np.random.default_rng(125 + m).standard_normal((m, n), dtype=np.float32)
    print(f"split-K residual {NAMES[qtype]} m={m} {xdtype}", flush=True)
    outs = []
    for ws in (torch.empty(need, dtype=torch.uint8, device="cuda"),
               torch.empty(need, dtype=torch.uint8, device="cuda"),
               torch.empty(need - 1, dtype=torch.uint8, device="cuda"),
               None):
        resid = torch.from_numpy(r0.copy()).cuda()
        rb = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        gguf_gemv_residual(x, q, qtype, (n, k), resid, rb, workspace=ws)
        got = resid.cpu().numpy()
        check_close(got, r0.astype(np.float64) + ref, f"split residual {NAMES[qtype]} m={m}")
        assert np.array_equal(rb.float().cpu().numpy(), _bf16_round(got))
        outs.append(got)
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.gpu
@pytest.mark.parametrize("qtype,n,k,m", [(Q6_K, 4096, 14336, 16), (Q6_K, 4144, 14336, 9),
                                         (Q4_K, 4144, 12800, 16), (Q4_K, 4096, 14336, 11)])
def test_gemv_residual_split_k_runs(qtype, n, k, m):
    """The split launch at the down projection's size: 7 splits x 256-259
    row tiles dealt to the CUs in equal runs that cross split boundaries
    (and, at K = 12800 for Q4_K, a last split of two chunks): within the bar
    of the oracle, the same on every call."""
    from dracort_amd.kernels import gemv_residual_workspace_bytes, gguf_gemv_residual

    need = gemv_residual_workspace_bytes(qtype, m, n, k)
    assert need == ((k // 256 + 7) // 8) * m * n * 4
    blocks, w = quantized(qtype, n, k, 400 + m)
    q = torch.from_numpy(blocks).cuda()
    x = activations(m, k, 410 + m, torch.bfloat16).cuda()
    ref = matmul_ref.linear_ref(x.cpu().float().numpy(), w)
    r0 = np.random.default_rng(420 + m).standard_normal((m, n), dtype=np.float32)
    print(f"split-K runs {NAMES[qtype]} [{n},{k}] m={m}", flush=True)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(2):
        resid = torch.from_numpy(r0.copy()).cuda()
        rb = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        gguf_gemv_residual(x, q, qtype, (n, k), resid, rb, workspace=ws)
        got = resid.cpu().numpy()
        check_close(got, r0.astype(np.float64) + ref, f"split runs {NAMES[qtype]} [{n},{k}] m={m}")
        assert np.array_equal(rb.float().cpu().numpy(), _bf16_round(got))
        outs.append(got)
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("qtype", [Q8_0, Q4_0])
@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
def test_gemv_single_token_block_formats(qtype, xdtype):
    """One token over Q8_0 / Q4_0 rows of K <= 4096 (the block-format
    single-token kernel: activations in registers, lanes past K idle): ragged
    row counts, short rows, the bias, a three-matrix launch with bf16 copies,
    and the residual epilogue."""
    from dracort_amd.kernels import gguf_gemv_multi, gguf_gemv_residual

    for n, k in ((1000, 4096), (64, 256), (3000, 2048), (17, 4096)):
        print(f"single token {NAMES[qtype]} [{n},{k}] {xdtype}", flush=True)
        y, ref = _run(qtype, n, k, 1, xdtype, seed=n + k, bias=(n == 1000))
        check_close(y, ref, f"x1b {NAMES[qtype]} [{n},{k}] {xdtype}")

    k = 1024
    ns = (512, 128, 128)
    x = activations(1, k, 7, xdtype)
    qs, refs, outs, outs_b = [], [], [], []
    for i, n in enumerate(ns):
        blocks, w = quantized(qtype, n, k, 40 + i)
        qs.append((torch.from_numpy(blocks).cuda(), n))
        refs.append(matmul_ref.linear_ref(x.float().numpy(), w))
        outs.append(torch.full((1, n), float("nan"), device="cuda"))
        outs_b.append(torch.empty((1, n), device="cuda", dtype=torch.bfloat16))
    gguf_gemv_multi(x.cuda(), qs, qtype, k, outs, outs_b)
    for i in range(3):
        got = outs[i].cpu().numpy()
        check_close(got, refs[i], f"x1b multi {NAMES[qtype]} matrix {i}")
        assert np.array_equal(outs_b[i].float().cpu().numpy(), _bf16_round(got))

    r0 = np.random.default_rng(9).standard_normal((1, 512), dtype=np.float32)
    resid = torch.from_numpy(r0.copy()).cuda()
    rb = torch.empty((1, 512), device="cuda", dtype=torch.bfloat16)
    gguf_gemv_residual(x.cuda(), qs[0][0], qtype, (512, k), resid, rb)
    got = resid.cpu().numpy()
    check_close(got, r0.astype(np.float64) + refs[0], f"x1b residual {NAMES[qtype]}")
    assert np.array_equal(rb.float().cpu().numpy(), _bf16_round(got))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_gemv_float32_matrix_core(qtype):
    """Float32 activations at 2..8 rows over Q4_0 / Q8_0 (the 4 x 4 x 1
    float32 MFMA kernel: one 256-element K range per item, the wave's partial
    tiles added in LDS): every row count on short and ragged rows (K ranges
    cut inside, row counts off the 16-row tile), one to four tiles per
    workgroup, uneven K ranges per wave (K = 14336), a three-matrix launch with
    bf16 copies, the residual epilogue, and the same bits on a second call."""
    from dracort_amd.kernels import gguf_gemv_multi, gguf_gemv_residual

    for n, k in ((16, 64), (33, 320), (130, 1088)):
        for m in range(2, 9):
            print(f"mf32 {NAMES[qtype]} [{n},{k}] m={m}", flush=True)
            y, ref = _run(qtype, n, k, m, torch.float32, seed=n + k + m, bias=(m == 5))
            check_close(y, ref, f"mf32 {NAMES[qtype]} [{n},{k}] m={m}")
    for n, k, m in ((4100, 4096, 3), (4100, 4096, 8), (16000, 1024, 5), (9000, 512, 2), (1000, 14336, 7)):
        print(f"mf32 {NAMES[qtype]} [{n},{k}] m={m}", flush=True)
        y, ref = _run(qtype, n, k, m, torch.float32, seed=n + m)
        check_close(y, ref, f"mf32 {NAMES[qtype]} [{n},{k}] m={m}")

    k, m = 1024, 6
    ns = (512, 128, 128)
    mats = [quantized(qtype, n, k, 300 + i) for i, n in enumerate(ns)]
    x = activations(m, k, 310, torch.float32)
    ys = [torch.full((m, n), float("nan"), device="cuda") for n in ns]
    ybs = [torch.empty((m, n), device="cuda", dtype=torch.bfloat16) for n in ns]
    print(f"mf32 multi {NAMES[qtype]}", flush=True)
    gguf_gemv_multi(x.cuda(), [(torch.from_numpy(b).cuda(), n) for (b, _), n in zip(mats, ns)], qtype, k, ys, ybs)
    for i, ((_, w), n) in enumerate(zip(mats, ns)):
        got = ys[i].cpu().numpy()
        check_close(got, matmul_ref.linear_ref(x.numpy(), w), f"mf32 multi {i}")
        assert np.array_equal(ybs[i].float().cpu().numpy(), _bf16_round(got))

    for n, k, m in ((4096, 14336, 7), (500, 4096, 3)):
        blocks, w = quantized(qtype, n, k, 320 + m)
        q = torch.from_numpy(blocks).cuda()
        x = activations(m, k, 330 + m, torch.float32).cuda()
        ref = matmul_ref.linear_ref(x.cpu().numpy(), w)
        r0 = np.random.default_rng(340 + m).standard_normal((m, n), dtype=np.float32)
        print(f"mf32 residual {NAMES[qtype]} [{n},{k}] m={m}", flush=True)
        outs = []
        for _ in range(2):
            resid = torch.from_numpy(r0.copy()).cuda()
            rb = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
            gguf_gemv_residual(x, q, qtype, (n, k), resid, rb)
            got = resid.cpu().numpy()
            check_close(got, r0.astype(np.float64) + ref, f"mf32 residual {NAMES[qtype]} [{n},{k}] m={m}")
            assert np.array_equal(rb.float().cpu().numpy(), _bf16_round(got))
            outs.append(got)
        assert np.array_equal(outs[0], outs[1])
