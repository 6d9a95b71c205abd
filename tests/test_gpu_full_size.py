"""GPU parity at the benchmark's full sizes, against the fp64 oracle:

* the Q6_K lm_head GEMV, 128256 x 4096, at 1 and 16 bf16 activation rows (the
  oracle dequantizes 256 weight rows at a time);
* the Q4_K prefill GEMM at M = 2048 on both full shapes (14336 x 4096 and
  4096 x 14336), checked on a seeded subset of 256 token rows plus the first
  and the last;
* the Mixtral-8x7B-shaped MoE FFN with all eight experts (H = 4096,
  I = 14336, Q4_K, 64 tokens, top-2), the oracle dequantizing one expert at a
  time.

Weights are drawn and quantized on the device (N(0, 0.02), 1 % of rows x4, as
the benchmark makes them); the oracle reads the same packed bytes back."""

import numpy as np
import pytest
import torch

from oracle import gguf_ref, matmul_ref
from tests.gguf_cases import Q4_K, Q6_K, check_close

pytestmark = pytest.mark.gpu


def _weight(n, k, qtype, seed):
    from dracort_amd.runtime.decode import synthetic_weight

    gen = torch.Generator(device="cuda").manual_seed(seed)
    return synthetic_weight(n, k, qtype, gen, "cuda")


def _linear_ref_chunked(qtype, blocks, n, k, x, rows=None, chunk=256):
    """fp64 x @ W.T from the oracle's dequantization, ``chunk`` weight rows at a time
    (``rows``: only these token rows of x)."""
    rb = gguf_ref.row_bytes(qtype, k)
    xs = np.asarray(x if rows is None else x[rows], dtype=np.float64)
    out = np.empty((xs.shape[0], n), dtype=np.float64)
    for r0 in range(0, n, chunk):
        r1 = min(n, r0 + chunk)
        w = gguf_ref.dequantize_matrix(qtype, blocks[r0 * rb:r1 * rb], (r1 - r0, k))
        out[:, r0:r1] = xs @ w.astype(np.float64).T
    return out


@pytest.mark.parametrize("m", [1, 16])
def test_lm_head_q6k_full_vocab(m):
    from dracort_amd.kernels import gguf_gemv

    n, k = 128256, 4096
    w = _weight(n, k, Q6_K, 41)
    blocks = w.data.cpu().numpy()
    x = torch.from_numpy(np.random.default_rng(41 + m).standard_normal((m, k), dtype=np.float32)).to(torch.bfloat16)
    print(f"lm_head Q6_K [{n},{k}] m={m}", flush=True)
    y = gguf_gemv(x.cuda(), w.data, Q6_K, (n, k)).cpu().numpy()
    ref = _linear_ref_chunked(Q6_K, blocks, n, k, x.float().numpy())
    for r in range(m):
        e, nw = check_close(y[r], ref[r], f"lm_head m={m} row {r}")
    print(f"lm_head m={m}: last row elementwise {e:.2e}, normwise {nw:.2e}", flush=True)


@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
def test_prefill_gemm_q4k_m2048_full_shape(n, k):
    from dracort_amd.kernels import gguf_linear

    m = 2048
    w = _weight(n, k, Q4_K, 43 + n)
    blocks = w.data.cpu().numpy()
    x = torch.from_numpy(np.random.default_rng(n).standard_normal((m, k), dtype=np.float32)).to(torch.bfloat16)
    print(f"prefill GEMM Q4_K [{n},{k}] m={m}", flush=True)
    y = gguf_linear(x.cuda(), w.data, Q4_K, (n, k)).cpu().numpy()
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(7).choice(m, 256, replace=False)]))
    ref = _linear_ref_chunked(Q4_K, blocks, n, k, x.float().numpy(), rows=rows, chunk=2048)
    e, nw = check_close(y[rows], ref, f"gemm [{n},{k}] m={m}")
    print(f"gemm [{n},{k}] m={m}: {rows.size} rows, elementwise {e:.2e}, normwise {nw:.2e}", flush=True)


def test_moe_mixtral_shape_all_eight_experts():
    from dracort_amd.kernels import gguf_moe

    h, inter, ne, t = 4096, 14336, 8, 64
    ws = [[_weight(inter, h, Q4_K, 100 + 3 * e), _weight(inter, h, Q4_K, 101 + 3 * e),
           _weight(h, inter, Q4_K, 102 + 3 * e)] for e in range(ne)]
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((t, h), dtype=np.float32)).to(torch.bfloat16)
    logits = rng.standard_normal((t, ne), dtype=np.float32)
    print(f"moe Q4_K H={h} I={inter} E={ne} T={t}", flush=True)
    y = gguf_moe(x.cuda(), torch.from_numpy(logits).cuda(), [g.data for g, _, _ in ws],
                 [u.data for _, u, _ in ws], [d.data for _, _, d in ws], Q4_K, inter, top_k=2).cpu().numpy()
    host = [[wq.data.cpu().numpy() for wq in triple] for triple in ws]
    del ws
    torch.cuda.empty_cache()

    def experts():  # one expert's float32 weights at a time
        for g, u, d in host:
            yield (gguf_ref.dequantize_matrix(Q4_K, g, (inter, h)), gguf_ref.dequantize_matrix(Q4_K, u, (inter, h)),
                   gguf_ref.dequantize_matrix(Q4_K, d, (h, inter)))

    ref = matmul_ref.moe_ref(x.float().numpy(), logits, experts(), 2)
    idx, _ = matmul_ref.route_ref(logits, 2)
    assert np.unique(idx).size == ne, "every expert receives tokens"
    e, nw = check_close(y, ref, "moe mixtral 8 experts")
    print(f"moe 8 experts: elementwise {e:.2e}, normwise {nw:.2e}", flush=True)
