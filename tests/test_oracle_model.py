"""Pins oracle.model_ref (the fp64 restatement of the reference forward pass)
with checks that do not retype its formula: a single token's layer in closed
form (one key: attention returns the value of the head's kv group, so q, k
and RoPE drop out), prefix consistency of the causal mask, position 0 seeing
only itself, fused q/k/v equal to split ones, tied embeddings, a MoE layer
against the dense FFN it reduces to with one expert, and planted mistakes
that these checks catch."""

import numpy as np

from oracle import decode_ref, matmul_ref, model_ref


def _weights(rng, hidden=16, heads=4, kv_heads=2, inter=24, vocab=20, layers=1, experts=0):
    d = hidden // heads
    w = {"token_embd.weight": rng.standard_normal((vocab, hidden)) * 0.5,
         "output_norm.weight": 1 + 0.1 * rng.standard_normal(hidden),
         "output.weight": rng.standard_normal((vocab, hidden)) * 0.3}
    for i in range(layers):
        p = f"blk.{i}."
        w[p + "attn_norm.weight"] = 1 + 0.1 * rng.standard_normal(hidden)
        w[p + "ffn_norm.weight"] = 1 + 0.1 * rng.standard_normal(hidden)
        w[p + "attn_q.weight"] = rng.standard_normal((heads * d, hidden)) * 0.3
        w[p + "attn_k.weight"] = rng.standard_normal((kv_heads * d, hidden)) * 0.3
        w[p + "attn_v.weight"] = rng.standard_normal((kv_heads * d, hidden)) * 0.3
        w[p + "attn_output.weight"] = rng.standard_normal((hidden, heads * d)) * 0.3
        if experts:
            w[p + "ffn_gate_inp.weight"] = rng.standard_normal((experts, hidden))
            w[p + "ffn_gate_exps.weight"] = rng.standard_normal((experts, inter, hidden)) * 0.3
            w[p + "ffn_up_exps.weight"] = rng.standard_normal((experts, inter, hidden)) * 0.3
            w[p + "ffn_down_exps.weight"] = rng.standard_normal((experts, hidden, inter)) * 0.3
        else:
            w[p + "ffn_gate.weight"] = rng.standard_normal((inter, hidden)) * 0.3
            w[p + "ffn_up.weight"] = rng.standard_normal((inter, hidden)) * 0.3
            w[p + "ffn_down.weight"] = rng.standard_normal((hidden, inter)) * 0.3
    return w


SPEC = model_ref.ModelSpec(hidden=16, layers=1, heads=4, kv_heads=2, eps=1e-6, theta=10000.0)


def _rms(x, g, eps=1e-6):
    return x / np.sqrt(np.mean(x * x) + eps) * g


def test_single_token_layer_in_closed_form():
    w = _weights(np.random.default_rng(0))
    tok = 7
    h0 = w["token_embd.weight"][tok]
    x0 = _rms(h0, w["blk.0.attn_norm.weight"])
    v = (w["blk.0.attn_v.weight"] @ x0).reshape(2, 4)
    att = np.concatenate([v[h // 2] for h in range(4)])  # one key: each head gets its group's value
    h1 = h0 + w["blk.0.attn_output.weight"] @ att
    x1 = _rms(h1, w["blk.0.ffn_norm.weight"])
    g, u = w["blk.0.ffn_gate.weight"] @ x1, w["blk.0.ffn_up.weight"] @ x1
    h2 = h1 + w["blk.0.ffn_down.weight"] @ (g / (1 + np.exp(-g)) * u)
    expect = w["output.weight"] @ _rms(h2, w["output_norm.weight"])
    got = model_ref.llama_forward(w, SPEC, [tok])[0]
    assert np.allclose(got, expect, rtol=1e-12, atol=1e-12)
    # q and k cannot matter for one token
    w2 = dict(w)
    w2["blk.0.attn_q.weight"] = w["blk.0.attn_q.weight"] * 3.0
    w2["blk.0.attn_k.weight"] = -w["blk.0.attn_k.weight"]
    assert np.allclose(model_ref.llama_forward(w2, SPEC, [tok])[0], expect, rtol=1e-12, atol=1e-12)
    # planted mistake: the residual of the attention block dropped
    wrong = w["output.weight"] @ _rms(h2 - h0, w["output_norm.weight"])
    assert not np.allclose(got, wrong, rtol=1e-6)


def test_prefix_consistency_of_the_causal_mask():
    w = _weights(np.random.default_rng(1), layers=2)
    spec = model_ref.ModelSpec(hidden=16, layers=2, heads=4, kv_heads=2, eps=1e-6)
    prompt = [3, 9, 1, 14, 5]
    full = model_ref.llama_forward(w, spec, prompt)
    for t in range(1, len(prompt) + 1):
        assert np.allclose(model_ref.llama_forward(w, spec, prompt[:t])[-1], full[t - 1], rtol=1e-11, atol=1e-11)


def test_causal_attention_position_zero_and_mask():
    rng = np.random.default_rng(2)
    q, k, v = rng.standard_normal((5, 4, 8)), rng.standard_normal((5, 2, 8)), rng.standard_normal((5, 2, 8))
    out = model_ref.causal_attention(q, k, v)
    for h in range(4):
        assert np.allclose(out[0, h], v[0, h // 2])  # position 0 sees only itself
    # the last row equals decode attention over the whole cache (the decode oracle, pinned separately)
    last = decode_ref.decode_attention_f64(q[-1], k.transpose(1, 0, 2), v.transpose(1, 0, 2), 5)
    assert np.allclose(out[-1], last, rtol=1e-12)
    # planted mistake: no mask -> row 0 differs
    s = np.einsum("hd,khd->hk", q[0], np.repeat(k, 2, axis=1)) / np.sqrt(8)
    p = np.exp(s - s.max(1, keepdims=True))
    unmasked = np.einsum("hk,khd->hd", p / p.sum(1, keepdims=True), np.repeat(v, 2, axis=1))
    assert not np.allclose(unmasked, out[0])


def test_fused_qkv_and_tied_embeddings():
    w = _weights(np.random.default_rng(3), layers=1)
    prompt = [2, 4, 6]
    split = model_ref.llama_forward(w, SPEC, prompt)
    fused = dict(w)
    fused["blk.0.attn_qkv.weight"] = np.concatenate(
        [w["blk.0.attn_q.weight"], w["blk.0.attn_k.weight"], w["blk.0.attn_v.weight"]])
    for s in "qkv":
        del fused[f"blk.0.attn_{s}.weight"]
    assert np.allclose(model_ref.llama_forward(fused, SPEC, prompt), split, rtol=1e-12, atol=1e-12)
    tied = dict(w)
    tied["output.weight"] = w["token_embd.weight"]
    spec_t = model_ref.ModelSpec(hidden=16, layers=1, heads=4, kv_heads=2, eps=1e-6, tied=True)
    assert np.allclose(model_ref.llama_forward(w, spec_t, prompt), model_ref.llama_forward(tied, SPEC, prompt))


def test_moe_layer_with_one_expert_is_the_dense_ffn():
    """Top-1 routing over one expert gives weight 1: the MoE layer reduces to that expert's dense FFN."""
    w = _weights(np.random.default_rng(4), experts=1)
    spec = model_ref.ModelSpec(hidden=16, layers=1, heads=4, kv_heads=2, eps=1e-6, experts=1, top_k=1)
    dense = {k: v for k, v in w.items() if "_exps" not in k and "gate_inp" not in k}
    for s in ("gate", "up", "down"):
        dense[f"blk.0.ffn_{s}.weight"] = w[f"blk.0.ffn_{s}_exps.weight"][0]
    prompt = [1, 2, 3]
    assert np.allclose(model_ref.llama_forward(w, spec, prompt), model_ref.llama_forward(dense, SPEC, prompt),
                       rtol=1e-12, atol=1e-12)
    # two experts, top-2: the layer output is the routing-weighted sum of both FFNs (route_ref pinned separately)
    w2 = _weights(np.random.default_rng(5), experts=2)
    spec2 = model_ref.ModelSpec(hidden=16, layers=1, heads=4, kv_heads=2, eps=1e-6, experts=2, top_k=2)
    out = model_ref.llama_forward(w2, spec2, [5])
    idx, rw = matmul_ref.route_ref(np.array([w2["blk.0.ffn_gate_inp.weight"] @ _rms(
        w2["token_embd.weight"][5] + w2["blk.0.attn_output.weight"] @ np.concatenate(
            [(w2["blk.0.attn_v.weight"] @ _rms(w2["token_embd.weight"][5], w2["blk.0.attn_norm.weight"]))
             .reshape(2, 4)[h // 2] for h in range(4)]), w2["blk.0.ffn_norm.weight"])]), 2)
    assert np.isclose(rw.sum(), 1.0) and set(idx[0]) == {0, 1}
    assert out.shape == (1, 20) and np.all(np.isfinite(out))


def test_float16_cache_rounding_changes_only_kv():
    """kv_dtype rounds the cached keys / values: one token's logits move by at
    most the float16 rounding of its value vector's effect, and do move."""
    w = _weights(np.random.default_rng(6))
    a = model_ref.llama_forward(w, SPEC, [3, 8, 11])
    b = model_ref.llama_forward(w, SPEC, [3, 8, 11], kv_dtype=np.float16)
    rel = np.max(np.abs(a - b)) / np.max(np.abs(a))
    assert 0 < rel < 1e-2
