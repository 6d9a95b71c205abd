"""GPU parity for Q4_1 / Q5_0 / Q5_1 / Q8_K / Q2_K / Q3_K / Q5_K (and the
upstream field order of Q2_K / Q3_K): bit-exact dequantization against the
oracle, and the fused GEMV / GEMM / MoE paths against the oracle's fp64
dequant-then-matmul (max elementwise relative error <= 1e-3)."""

import numpy as np
import pytest
import torch

from dracort_amd.kernels import (
    gguf_dequantize,
    gguf_gemm,
    gguf_gemv,
    gguf_gemv_multi,
    gguf_gemv_residual,
    gguf_gemv_swiglu,
    gguf_moe,
)
from oracle import gguf_ref, matmul_ref
from tests.gguf_cases import (
    GGML_ORDER,
    MORE_TYPES,
    Q2_K,
    Q3_K,
    Q4_1,
    Q5_K,
    activations,
    check_close,
    qk_of,
    quantized,
    type_name,
)

pytestmark = pytest.mark.gpu

F16_FIELDS = {3: [0, 2], 6: [0], 7: [0, 2], 15: [0], 10: [0, 2], 11: [0], 13: [0, 2]}
ORDERED = [Q2_K, Q3_K, Q2_K | GGML_ORDER, Q3_K | GGML_ORDER]


def _dev(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).reshape(-1)).cuda()


def _random_blocks(qtype, nb, seed):
    """Random bytes, float16 fields finite (normal, wide, subnormal, +-0, extremes)."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nb, gguf_ref.BLOCK_LAYOUT[qtype][1]), dtype=np.uint8)
    special = np.array([0x0000, 0x8000, 0x7BFF, 0xFBFF, 0x0400, 0x0001], dtype=np.uint16)
    for off in F16_FIELDS[qtype]:
        bits = (rng.normal(size=nb) * 0.05).astype(np.float16).view(np.uint16).copy()
        kind = rng.integers(0, 4, size=nb)
        bits[kind == 1] = (rng.normal(size=nb) * 500).astype(np.float16).view(np.uint16)[kind == 1]
        bits[kind == 2] = rng.integers(1, 0x400, size=nb, dtype=np.uint16)[kind == 2]
        bits[kind == 3] = special[rng.integers(0, special.size, size=nb)][kind == 3]
        b[:, off] = (bits & 0xFF).astype(np.uint8)
        b[:, off + 1] = (bits >> 8).astype(np.uint8)
    return b


@pytest.mark.parametrize("qtype", MORE_TYPES)
def test_dequant_random_blocks_bit_exact(qtype):
    qk = qk_of(qtype)
    nb = 192 if qk == 32 else 48
    blocks = _random_blocks(qtype, nb, seed=qtype)
    expect = gguf_ref.dequantize(qtype, blocks, nb * qk).view(np.uint32)
    # one row, and rows of one block (2-byte aligned rows for Q5_0 / Q3_K / Q8_K)
    for n, k in ((1, nb * qk), (nb, qk)):
        print(f"dequant {type_name(qtype)} [{n},{k}]", flush=True)
        got = gguf_dequantize(_dev(blocks), qtype, (n, k)).cpu().numpy()
        assert np.array_equal(got.reshape(-1).view(np.uint32), expect), (type_name(qtype), n, k)
    if qtype in (Q2_K, Q3_K):
        up = gguf_ref.to_ggml_order(qtype, blocks)
        got = gguf_dequantize(_dev(up), qtype | GGML_ORDER, (nb, qk)).cpu().numpy()
        assert np.array_equal(got.reshape(-1).view(np.uint32), expect)


@pytest.mark.parametrize("qtype", MORE_TYPES + [Q2_K | GGML_ORDER, Q3_K | GGML_ORDER])
def test_dequant_quantized_weight_bit_exact(qtype):
    for n, k in ((4096, 4096), (3, 768)):
        print(f"dequant {type_name(qtype)} [{n},{k}]", flush=True)
        blocks, ref = quantized(qtype, n, k, seed=n + k)
        got = gguf_dequantize(_dev(blocks), qtype, (n, k)).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (type_name(qtype), n, k)


def _gemv(qtype, n, k, m, xdtype, seed):
    blocks, w = quantized(qtype, n, k, seed)
    x = activations(m, k, seed, xdtype)
    ref = matmul_ref.linear_ref(x.float().numpy(), w)
    y = gguf_gemv(x.cuda(), torch.from_numpy(blocks).cuda(), qtype, (n, k)).cpu().numpy()
    return y, ref


@pytest.mark.parametrize("qtype", MORE_TYPES + [Q2_K | GGML_ORDER, Q3_K | GGML_ORDER])
def test_gemv_llama_shapes(qtype):
    for n, k in ((4096, 4096), (14336, 4096), (4096, 14336)):
        for m, xd in ((1, torch.bfloat16), (1, torch.float32), (4, torch.bfloat16), (16, torch.float32)):
            print(f"gemv {type_name(qtype)} [{n},{k}] m={m} {xd}", flush=True)
            y, ref = _gemv(qtype, n, k, m, xd, seed=n % 97 + m)
            check_close(y, ref, f"gemv {type_name(qtype)} [{n},{k}] m={m} {xd}")


@pytest.mark.parametrize("qtype", MORE_TYPES)
def test_gemv_ragged_shapes_every_tile(qtype):
    qk = qk_of(qtype)
    for n, k in ((1, qk), (7, 3 * qk), (33, 5 * qk), (130, 2 * qk)):
        for m in (1, 2, 3, 5, 9, 16):
            xd = torch.bfloat16 if m % 2 else torch.float32
            print(f"gemv {type_name(qtype)} [{n},{k}] m={m}", flush=True)
            y, ref = _gemv(qtype, n, k, m, xd, seed=n * 31 + m)
            check_close(y, ref, f"gemv {type_name(qtype)} [{n},{k}] m={m}")


@pytest.mark.parametrize("qtype", [Q5_K, Q3_K, Q4_1])
def test_fused_decode_launches(qtype):
    """multi (q, k, v), SwiGLU and residual modes of the decode GEMV."""
    h, i = 1024, 2048
    x = activations(2, h, qtype, torch.bfloat16)
    xd = x.cuda()
    xs = x.float().numpy()
    mats = [quantized(qtype, n, h, seed=qtype + j) for j, n in enumerate((1024, 256, 256))]
    outs = [torch.empty((2, n), dtype=torch.float32, device="cuda") for n in (1024, 256, 256)]
    print(f"multi {type_name(qtype)}", flush=True)
    gguf_gemv_multi(xd, [(torch.from_numpy(b).cuda(), w.shape[0]) for b, w in mats], qtype, h, outs)
    for (b, w), y in zip(mats, outs):
        check_close(y.cpu().numpy(), matmul_ref.linear_ref(xs, w), f"multi {type_name(qtype)}")
    gb, gw = quantized(qtype, i, h, seed=qtype + 5)
    ub, uw = quantized(qtype, i, h, seed=qtype + 6)
    print(f"swiglu {type_name(qtype)}", flush=True)
    y = torch.empty((2, i), dtype=torch.float32, device="cuda")
    gguf_gemv_swiglu(xd, torch.from_numpy(gb).cuda(), torch.from_numpy(ub).cuda(), qtype, (i, h), out=y)
    g = matmul_ref.linear_ref(xs, gw)
    ref = g / (1.0 + np.exp(-g)) * matmul_ref.linear_ref(xs, uw)
    check_close(y.cpu().numpy(), ref, f"swiglu {type_name(qtype)}")
    db, dw = quantized(qtype, h, i, seed=qtype + 7)
    s = activations(2, i, qtype + 8, torch.bfloat16)
    resid = torch.from_numpy(np.random.default_rng(qtype).standard_normal((2, h), dtype=np.float32))
    rd = resid.cuda()
    print(f"residual {type_name(qtype)}", flush=True)
    gguf_gemv_residual(s.cuda(), torch.from_numpy(db).cuda(), qtype, (h, i), rd)
    ref = resid.numpy().astype(np.float64) + matmul_ref.linear_ref(s.float().numpy(), dw)
    check_close(rd.cpu().numpy(), ref, f"residual {type_name(qtype)}")


@pytest.mark.parametrize("qtype", MORE_TYPES + [Q2_K | GGML_ORDER, Q3_K | GGML_ORDER])
def test_gemm_tile_edges(qtype):
    qk = qk_of(qtype)
    for n, k, m in ((1, qk, 17), (130, 2 * qk, 129), (257, 3 * qk, 40)):
        print(f"gemm {type_name(qtype)} [{n},{k}] m={m}", flush=True)
        blocks, w = quantized(qtype, n, k, seed=n + m)
        x = activations(m, k, n + m, torch.bfloat16)
        y = gguf_gemm(x.cuda(), torch.from_numpy(blocks).cuda(), qtype, (n, k)).cpu().numpy()
        check_close(y, matmul_ref.linear_ref(x.float().numpy(), w), f"gemm {type_name(qtype)} [{n},{k}] m={m}")


def test_gemm_q5k_prefill_shape():
    blocks, w = quantized(Q5_K, 14336, 4096, seed=2)
    x = activations(512, 4096, 2, torch.bfloat16)
    print("gemm Q5_K [14336,4096] m=512", flush=True)
    y = gguf_gemm(x.cuda(), torch.from_numpy(blocks).cuda(), Q5_K, (14336, 4096)).cpu().numpy()
    check_close(y, matmul_ref.linear_ref(x.float().numpy(), w), "gemm Q5_K m=512")


@pytest.mark.parametrize("qtype", [Q5_K, Q2_K, Q4_1])
def test_moe_top2(qtype):
    t, h, i, e = 48, 512, 768 if qtype == Q4_1 else 1024, 4
    ex = [tuple(quantized(qtype, *shape, seed=qtype + 3 * j + r) for r, shape in enumerate(((i, h), (i, h), (h, i))))
          for j in range(e)]
    x = activations(t, h, qtype, torch.bfloat16)
    logits = np.random.default_rng(qtype).standard_normal((t, e), dtype=np.float32)
    ref = matmul_ref.moe_ref(x.float().numpy(), logits, [(g[1], u[1], d[1]) for g, u, d in ex], 2)
    dev = lambda b: torch.from_numpy(b[0]).cuda()  # noqa: E731
    print(f"moe {type_name(qtype)} T={t} E={e}", flush=True)
    y = gguf_moe(x.cuda(), torch.from_numpy(logits).cuda(), [dev(g) for g, _, _ in ex],
                 [dev(u) for _, u, _ in ex], [dev(d) for _, _, d in ex], qtype, i, top_k=2).cpu().numpy()
    check_close(y, ref, f"moe {type_name(qtype)}")
