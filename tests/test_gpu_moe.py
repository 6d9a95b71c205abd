"""GPU parity: sparse MoE FFN (device routing + grouped GGUF expert GEMVs +
weighted combine) against the oracle's fp64 closed form, <= 1e-3."""

import numpy as np
import pytest
import torch

from dracort_amd.kernels import gguf_moe
from oracle import matmul_ref
from tests.gguf_cases import NAMES, Q4_0, Q4_K, Q6_K, Q8_0, activations, check_close, quantized

pytestmark = pytest.mark.gpu


def _experts(qtype, e, h, i, seed):
    out = []
    for j in range(e):
        g = quantized(qtype, i, h, seed + 3 * j)
        u = quantized(qtype, i, h, seed + 3 * j + 1)
        d = quantized(qtype, h, i, seed + 3 * j + 2)
        out.append((g, u, d))
    return out


def _run(qtype, t, h, i, e, k, seed, logits=None, xdtype=torch.bfloat16):
    ex = _experts(qtype, e, h, i, seed)
    x = activations(t, h, seed, xdtype)
    if logits is None:
        logits = np.random.default_rng(seed).standard_normal((t, e), dtype=np.float32)
    ref = matmul_ref.moe_ref(x.float().numpy(), logits, [(g[1], u[1], d[1]) for g, u, d in ex], k)
    dev = lambda b: torch.from_numpy(b[0]).cuda()  # noqa: E731
    y = gguf_moe(
        x.cuda(), torch.from_numpy(logits).cuda(),
        [dev(g) for g, _, _ in ex], [dev(u) for _, u, _ in ex], [dev(d) for _, _, d in ex],
        qtype, i, top_k=k,
    ).cpu().numpy()
    return y, ref


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q8_0, Q4_0])
def test_moe_top2_8_experts(qtype):
    print(f"moe {NAMES[qtype]} T=64 E=8", flush=True)
    y, ref = _run(qtype, 64, 512, 1024, 8, 2, seed=qtype)
    check_close(y, ref, f"moe {NAMES[qtype]}")


def test_moe_edge_routing():
    # a single token
    y, ref = _run(Q4_K, 1, 256, 512, 4, 2, seed=21)
    check_close(y, ref, "moe T=1")
    # every token routed to experts 2 and 3 (one expert gets > 16 tokens: several M tiles)
    t = 40
    logits = np.full((t, 4), -5.0, dtype=np.float32)
    logits[:, 2] = 3.0
    logits[:, 3] = np.linspace(-1, 1, t, dtype=np.float32)
    y, ref = _run(Q4_K, t, 256, 512, 4, 2, seed=22, logits=logits)
    check_close(y, ref, "moe skewed")
    # top-1 routing, float32 activations
    y, ref = _run(Q8_0, 33, 256, 256, 5, 1, seed=23, xdtype=torch.float32)
    check_close(y, ref, "moe top1 f32")


def test_moe_route_paths():
    """Up to 256 tokens are routed one per thread (one ballot per expert and
    wave), more by the general grouping loop; both against the oracle, with
    ties in the logits (rounded to 0.5: equal logits go to the lower expert),
    up to 64 experts and top-8."""
    for t, e, k in ((256, 16, 4), (300, 8, 2), (130, 64, 8)):
        logits = (np.round(np.random.default_rng(40 + t).standard_normal((t, e)) * 2) / 2).astype(np.float32)
        print(f"moe routing T={t} E={e} k={k}", flush=True)
        y, ref = _run(Q4_K, t, 256, 512, e, k, seed=41 + e, logits=logits)
        check_close(y, ref, f"moe routing T={t} E={e} k={k}")


@pytest.mark.parametrize("qtype", [Q4_K, Q4_0])
def test_moe_matrix_core_f32(qtype):
    """float32 hidden states on the matrix-core experts (three bf16 planes),
    ragged per-expert counts (33 tokens, top-2 over 5 experts)."""
    print(f"moe {NAMES[qtype]} f32 T=33 E=5", flush=True)
    y, ref = _run(qtype, 33, 512, 768, 5, 2, seed=24 + qtype, xdtype=torch.float32)
    check_close(y, ref, f"moe {NAMES[qtype]} f32")


def test_moe_mixtral_shape_subset():
    """Mixtral-8x7B expert shapes (H=4096, I=14336), Q4_K, 64 tokens, top-2;
    two experts so the fp64 oracle stays small."""
    print("moe Q4_K H=4096 I=14336 E=2 T=64", flush=True)
    y, ref = _run(Q4_K, 64, 4096, 14336, 2, 2, seed=31)
    check_close(y, ref, "moe mixtral-shape")
