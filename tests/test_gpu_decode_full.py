"""GPU parity of the full decode step (RMSNorm, q/k/v, RoPE + KV-cache append
+ attention, o_proj + residual, RMSNorm, SwiGLU, down + residual, final norm,
lm_head) against an fp64 oracle chain with the same rounding points (bf16
GEMV inputs, float16 cache entries), over several consecutive tokens."""

import numpy as np
import pytest
import torch

from oracle import decode_ref, gguf_ref, matmul_ref

pytestmark = pytest.mark.gpu


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy().astype(np.float64)


def _setup(m, start):
    from dracort_amd.runtime.decode import AttentionShape, DecodeStep, LlamaShape, synthetic_layer_set

    shape = LlamaShape(hidden=512, inter=1024, kv_dim=128, vocab=1024, n_layers=2)
    ls = synthetic_layer_set(shape, seed=5, device="cuda")
    attn = AttentionShape(n_heads=8, n_kv_heads=2, head_dim=64, rope_theta=10000.0, rms_eps=1e-5, max_positions=64)
    step = DecodeStep(ls, m=m, attention=attn, start_position=start)
    gen = torch.Generator(device="cuda").manual_seed(9)
    for kc, vc in zip(step.k_cache, step.v_cache):  # tokens already in the caches
        kc[:, :, :start] = torch.randn(kc[:, :, :start].shape, generator=gen, device="cuda").half()
        vc[:, :, :start] = torch.randn(vc[:, :, :start].shape, generator=gen, device="cuda").half()
    return ls, attn, step


def _oracle_step(ls, attn, x, kcs, vcs, positions):
    """One step for m sequences in fp64; kcs / vcs (numpy float16, updated in place)."""
    def w(qw):
        return gguf_ref.dequantize_matrix(qw.ggml_type, qw.data.cpu().numpy(), qw.shape).astype(np.float64)

    hd, hq, hkv = attn.head_dim, attn.n_heads, attn.n_kv_heads
    cos, sin = decode_ref.rope_tables(hd, np.arange(attn.max_positions), attn.rope_theta)
    h = x.astype(np.float64)
    for li, layer in enumerate(ls.layers):
        nw = {k: v.cpu().numpy() for k, v in ls.norms[li].items()}
        xn = _bf16(decode_ref.rms_norm_f64(h, nw["attn"], attn.rms_eps))
        q = (xn @ w(layer["q"]).T).astype(np.float32)
        k = (xn @ w(layer["k"]).T).astype(np.float32)
        v = (xn @ w(layer["v"]).T).astype(np.float32)
        att = np.empty_like(h)
        for b, p in enumerate(positions):
            c, s = cos[p].astype(np.float64), sin[p].astype(np.float64)
            qr = decode_ref.apply_rope(q[b].reshape(hq, hd).astype(np.float64), c, s)
            kr = decode_ref.apply_rope(k[b].reshape(hkv, hd).astype(np.float64), c, s)
            kcs[li][b, :, p] = kr.astype(np.float16)
            vcs[li][b, :, p] = v[b].reshape(hkv, hd).astype(np.float16)
            att[b] = decode_ref.decode_attention_f64(qr, kcs[li][b], vcs[li][b], p + 1).reshape(-1)
        h = h + _bf16(att) @ w(layer["o"]).T
        xn = _bf16(decode_ref.rms_norm_f64(h, nw["ffn"], attn.rms_eps))
        g = xn @ w(layer["gate"]).T
        u = xn @ w(layer["up"]).T
        h = h + _bf16(matmul_ref.silu64(g) * u) @ w(layer["down"]).T
    xn = _bf16(decode_ref.rms_norm_f64(h, ls.output_norm.cpu().numpy(), attn.rms_eps))
    return xn @ w(ls.lm_head).T


@pytest.mark.parametrize("m", [1, 3])
def test_full_decode_steps_match_oracle_chain(m):
    start = 5
    ls, attn, step = _setup(m, start)
    kcs = [kc.cpu().numpy() for kc in step.k_cache]
    vcs = [vc.cpu().numpy() for vc in step.v_cache]
    x = step.x_in.float().cpu().numpy()
    for t in range(3):
        print(f"full decode m={m} step {t}", flush=True)
        got = step.run().cpu().numpy()
        ref = _oracle_step(ls, attn, x, kcs, vcs, [start + t] * m)
        elem, norm = matmul_ref.rel_err(got, ref)
        # bf16 roundings of intermediate activations can land on the other side of a
        # rounding boundary, so the chain is held to a normwise bound
        assert norm < 3e-3, (t, elem, norm)
        assert step.positions.cpu().tolist() == [start + t + 1] * m
        for li in range(len(ls.layers)):
            got_k = step.k_cache[li][:, :, start + t].float().cpu().numpy()
            ref_k = kcs[li][:, :, start + t].astype(np.float32)
            assert np.max(np.abs(got_k - ref_k)) <= 2 * np.max(np.abs(np.spacing(ref_k.astype(np.float16)))) + 1e-3


def test_full_decode_graph_replays_advance_positions():
    ls, attn, step = _setup(1, 2)
    step.capture()  # the capture itself runs one eager warm-up step (position 2) first
    torch.cuda.synchronize()
    start = int(step.positions.item())
    outs = []
    for i in range(3):
        print(f"full decode replay {i}", flush=True)
        outs.append(step.replay().clone())
        torch.cuda.synchronize()
    assert int(step.positions.item()) == start + 3
    assert not torch.equal(outs[0], outs[1])  # a new token each replay
    assert all(torch.isfinite(o).all() for o in outs)
