"""GPU parity of the fused decode launches (q/k/v in one launch, gate/up with
SwiGLU, projection + residual add) against the oracle, the decode chain
against an fp64 restatement of the same chain, and HIP-graph replays against
eager execution."""

import numpy as np
import pytest
import torch

from dracort_amd.kernels import gguf_gemv_multi, gguf_gemv_residual, gguf_gemv_swiglu
from oracle import gguf_ref, matmul_ref
from tests.gguf_cases import Q4_K, Q6_K, Q8_0, activations, check_close, quantized

pytestmark = pytest.mark.gpu


def _bf16_round(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def test_gemv_multi_uneven_row_split():
    """Row ranges of very different sizes (the mapping from launch row to
    (matrix, row) must stop at the owning matrix)."""
    ns = (10, 300, 7, 1500)
    mats = [quantized(Q4_K, n, 1024, seed=70 + i) for i, n in enumerate(ns)]
    x = activations(2, 1024, 70, torch.bfloat16)
    outs = [torch.full((2, n), float("nan"), device="cuda") for n in ns]
    gguf_gemv_multi(x.cuda(), [(torch.from_numpy(b).cuda(), n) for (b, _), n in zip(mats, ns)], Q4_K, 1024, outs)
    for (b, w), o in zip(mats, outs):
        check_close(o.cpu().numpy(), matmul_ref.linear_ref(x.float().numpy(), w), "uneven multi")


@pytest.mark.parametrize("m", [1, 3, 8])
def test_gemv_multi_qkv(m):
    mats = [quantized(Q4_K, n, 4096, seed=40 + i) for i, n in enumerate((4096, 1024, 1024))]
    x = activations(m, 4096, 40 + m, torch.bfloat16)
    xd = x.cuda()
    outs = [torch.empty((m, n), device="cuda") for n in (4096, 1024, 1024)]
    outs_b = [torch.empty((m, n), device="cuda", dtype=torch.bfloat16) for n in (4096, 1024, 1024)]
    gguf_gemv_multi(xd, [(torch.from_numpy(b).cuda(), w.shape[0]) for b, w in mats], Q4_K, 4096, outs, outs_b)
    for (b, w), o, ob in zip(mats, outs, outs_b):
        ref = matmul_ref.linear_ref(x.float().numpy(), w)
        y = o.cpu().numpy()
        check_close(y, ref, f"qkv m={m}")
        assert np.array_equal(ob.float().cpu().numpy(), _bf16_round(y))


@pytest.mark.parametrize("qtype,n,k", [(Q4_K, 14336, 4096), (Q6_K, 512, 1024), (Q8_0, 300, 512)])
@pytest.mark.parametrize("m", [1, 4, 16])
def test_gemv_swiglu(qtype, n, k, m):
    bg, wg = quantized(qtype, n, k, seed=50)
    bu, wu = quantized(qtype, n, k, seed=51)
    x = activations(m, k, 50 + m, torch.bfloat16)
    g = matmul_ref.linear_ref(x.float().numpy(), wg)
    u = matmul_ref.linear_ref(x.float().numpy(), wu)
    ref = matmul_ref.silu64(g) * u
    y = torch.empty((m, n), device="cuda")
    yb = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
    gguf_gemv_swiglu(x.cuda(), torch.from_numpy(bg).cuda(), torch.from_numpy(bu).cuda(), qtype, (n, k), y, yb)
    check_close(y.cpu().numpy(), ref, f"swiglu m={m}")
    assert np.array_equal(yb.float().cpu().numpy(), _bf16_round(y.cpu().numpy()))


@pytest.mark.parametrize("qtype,n,k", [(Q6_K, 4096, 14336), (Q4_K, 4096, 4096), (Q4_K, 130, 512)])
@pytest.mark.parametrize("m,xdtype", [(1, torch.bfloat16), (2, torch.float32), (16, torch.bfloat16)])
def test_gemv_residual(qtype, n, k, m, xdtype):
    b, w = quantized(qtype, n, k, seed=60)
    x = activations(m, k, 60 + m, xdtype)
    r0 = np.random.default_rng(61).standard_normal((m, n), dtype=np.float32)
    ref = r0.astype(np.float64) + matmul_ref.linear_ref(x.float().numpy(), w)
    resid = torch.from_numpy(r0.copy()).cuda()
    rb = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
    gguf_gemv_residual(x.cuda(), torch.from_numpy(b).cuda(), qtype, (n, k), resid, rb)
    got = resid.cpu().numpy()
    check_close(got, ref, f"residual m={m}")
    assert np.array_equal(rb.float().cpu().numpy(), _bf16_round(got))


def test_fused_entry_points_reject_aliasing():
    b, _ = quantized(Q4_K, 256, 256, seed=1)
    q = torch.from_numpy(b).cuda()
    buf = torch.empty(4096, device="cuda")
    x = buf[:256].view(1, 256)
    with pytest.raises(ValueError, match="overlap"):
        gguf_gemv_residual(x, q, Q4_K, (256, 256), buf[:256].view(1, 256))


# --- decode chain --------------------------------------------------------------

def _small_layer_set():
    from dracort_amd.runtime.decode import LlamaShape, synthetic_layer_set

    shape = LlamaShape(hidden=512, inter=1024, kv_dim=128, vocab=1024, n_layers=2)
    return synthetic_layer_set(shape, seed=3, device="cuda")


def _oracle_chain(ls, x_bf16: np.ndarray) -> np.ndarray:
    """fp64 chain with the launches' bf16 roundings at the same points."""
    def w(qw):
        return gguf_ref.dequantize_matrix(qw.ggml_type, qw.data.cpu().numpy(), qw.shape).astype(np.float64)

    h = x_bf16.astype(np.float64)
    hb = _bf16_round(h).astype(np.float64)
    for layer in ls.layers:
        q = _bf16_round(hb @ w(layer["q"]).T)
        h = h + q @ w(layer["o"]).T
        hb = _bf16_round(h)
        g = hb @ w(layer["gate"]).T
        u = hb @ w(layer["up"]).T
        s = _bf16_round(matmul_ref.silu64(g) * u)
        h = h + s @ w(layer["down"]).T
        hb = _bf16_round(h)
    return hb @ w(ls.lm_head).T


def test_decode_chain_matches_oracle_chain():
    from dracort_amd.runtime.decode import DecodeStep

    ls = _small_layer_set()
    step = DecodeStep(ls, m=2)
    got = step.run().cpu().numpy()
    ref = _oracle_chain(ls, step.x_in.float().cpu().numpy())
    elem, norm = matmul_ref.rel_err(got, ref)
    # bf16 roundings of intermediate activations can land on the other side of a
    # rounding boundary, so the chain is held to a normwise bound
    assert norm < 2e-3, (elem, norm)


def test_decode_graph_replays_match_eager():
    from dracort_amd.runtime.decode import DecodeStep

    ls = _small_layer_set()
    step = DecodeStep(ls, m=1)
    eager = step.run().clone()
    torch.cuda.synchronize()
    step.capture()
    scratch = torch.zeros(1 << 20, device="cuda")
    for i in range(4):
        scratch.add_(float(i))           # unrelated eager work between replays
        torch.cuda.synchronize()
        out = step.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from eager"
