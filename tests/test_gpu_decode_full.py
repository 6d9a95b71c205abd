"""GPU parity of the full decode step (RMSNorm, q/k/v, RoPE + KV-cache append
+ attention, o_proj + residual, RMSNorm, SwiGLU, down + residual, final norm,
lm_head) over several consecutive tokens, against two fp64 oracle chains:

* one with the step's own rounding points (bf16 GEMV inputs, float16 cache
  entries), held to 3e-3 normwise;
* one that keeps every activation and the cache unrounded, as the
  reference's ``forward_step`` does with its default float32 KV cache
  (``draco/runtime/cpu/executor.py:290-342``, ``kv_cache_dtype="f32"`` at
  ``:131-137``): the step's deviation from the reference chain, held to the
  reference's own end-to-end bar ``allclose(atol=1e-2, rtol=1e-2)``
  (``tests/format/test_gguf.py:762``)."""

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


def _oracle_step(ls, attn, x, kcs, vcs, positions, rounded=True):
    """One step for m sequences in fp64; kcs / vcs (numpy, updated in place).
    rounded: bf16 GEMV inputs and float16 cache entries as the step stores them;
    otherwise every activation and cache entry stays unrounded."""
    rb = _bf16 if rounded else (lambda a: np.asarray(a, dtype=np.float64))
    cdt = np.float16 if rounded else np.float64
    pdt = np.float32 if rounded else np.float64

    def w(qw):
        return gguf_ref.dequantize_matrix(qw.ggml_type, qw.data.cpu().numpy(), qw.shape).astype(np.float64)

    hd, hq, hkv = attn.head_dim, attn.n_heads, attn.n_kv_heads
    cos, sin = decode_ref.rope_tables(hd, np.arange(attn.max_positions), attn.rope_theta)
    h = x.astype(np.float64)
    for li, layer in enumerate(ls.layers):
        nw = {k: v.cpu().numpy() for k, v in ls.norms[li].items()}
        xn = rb(decode_ref.rms_norm_f64(h, nw["attn"], attn.rms_eps))
        q = (xn @ w(layer["q"]).T).astype(pdt)
        k = (xn @ w(layer["k"]).T).astype(pdt)
        v = (xn @ w(layer["v"]).T).astype(pdt)
        att = np.empty_like(h)
        for b, p in enumerate(positions):
            c, s = cos[p].astype(np.float64), sin[p].astype(np.float64)
            qr = decode_ref.apply_rope(q[b].reshape(hq, hd).astype(np.float64), c, s)
            kr = decode_ref.apply_rope(k[b].reshape(hkv, hd).astype(np.float64), c, s)
            kcs[li][b, :, p] = kr.astype(cdt)
            vcs[li][b, :, p] = v[b].reshape(hkv, hd).astype(cdt)
            att[b] = decode_ref.decode_attention_f64(qr, kcs[li][b], vcs[li][b], p + 1).reshape(-1)
        h = h + rb(att) @ w(layer["o"]).T
        xn = rb(decode_ref.rms_norm_f64(h, nw["ffn"], attn.rms_eps))
        g = xn @ w(layer["gate"]).T
        u = xn @ w(layer["up"]).T
        h = h + rb(matmul_ref.silu64(g) * u) @ w(layer["down"]).T
    xn = rb(decode_ref.rms_norm_f64(h, ls.output_norm.cpu().numpy(), attn.rms_eps))
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


@pytest.mark.parametrize("m", [1, 3])
def test_full_decode_steps_within_reference_bar_of_float32_chain(m):
    """Deviation of the step (bf16 activations between launches, float16 KV
    cache) from the reference's unrounded chain: elementwise and normwise
    figures printed, held to the reference's end-to-end bar."""
    start = 5
    ls, attn, step = _setup(m, start)
    kcs = [kc.cpu().numpy().astype(np.float64) for kc in step.k_cache]
    vcs = [vc.cpu().numpy().astype(np.float64) for vc in step.v_cache]
    x = step.x_in.float().cpu().numpy()
    for t in range(3):
        got = step.run().cpu().numpy()
        ref = _oracle_step(ls, attn, x, kcs, vcs, [start + t] * m, rounded=False)
        elem, norm = matmul_ref.rel_err(got, ref)
        worst = float(np.max(np.abs(got - ref) - 1e-2 * np.abs(ref)))
        print(f"full decode m={m} step {t} vs float32 chain: elementwise {elem:.3e}, normwise {norm:.3e}, "
              f"max |d| - 1e-2 |ref| = {worst:.3e} (max |ref| {np.max(np.abs(ref)):.3f})", flush=True)
        assert np.allclose(got, ref, atol=1e-2, rtol=1e-2), (t, elem, norm, worst)
        assert norm < 1e-2, (t, elem, norm)


def test_full_decode_graph_replays_advance_positions():
    ls, attn, step = _setup(1, 2)
    step.capture()  # the eager warm-up step inside capture() leaves the positions as they were
    torch.cuda.synchronize()
    start = int(step.positions.item())
    assert start == 2 and step.next_position == 2
    outs = []
    for i in range(3):
        print(f"full decode replay {i}", flush=True)
        outs.append(step.replay().clone())
        torch.cuda.synchronize()
    assert int(step.positions.item()) == start + 3
    assert not torch.equal(outs[0], outs[1])  # a new token each replay
    assert all(torch.isfinite(o).all() for o in outs)


def test_full_decode_refuses_a_step_past_the_cache():
    """The step that would write position max_positions raises before any launch."""
    from dracort_amd.exceptions import KVCacheError

    ls, attn, step = _setup(1, 61)  # max_positions 64: positions 61, 62, 63 fit
    for _ in range(3):
        step.run()
    torch.cuda.synchronize()
    assert int(step.positions.item()) == 64
    with pytest.raises(KVCacheError):
        step.run()
    assert int(step.positions.item()) == 64
