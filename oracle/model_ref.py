"""fp64 restatement of the reference executor's forward pass for the llama
family, plus a sparse-MoE FFN layer (oracle only).

Follows ``CPUExecutionBackend.forward_step`` (``draco/runtime/cpu/executor.py:290-342``)
with the pieces it calls:

* embedding rows ``embed[token_ids]`` (``_initial_hidden``, ``:279-288``);
* per layer: ``rms_norm`` (``draco/runtime/cpu/ops.py:15-19``), q / k / v
  projections with optional biases or one fused qkv projection split into
  q, k, v (``_qkv``, ``:243-271``), RoPE on q and k with the float32 tables of
  ``build_rope_cache`` (``ops.py:73-92``), causal attention over the cached
  keys with the kv heads repeated over their query-head groups
  (``draco/runtime/cpu/attention.py:35-81``), ``o_proj`` and the residual add,
  ``rms_norm``, ``down(silu(gate x) * up x)`` and the residual add (``_mlp``,
  ``:208-224``);
* the final ``rms_norm`` and the lm_head, or the embedding matrix when the
  embeddings are tied (``:331-339``).

A layer that carries experts instead of a dense MLP routes each token with
``matmul_ref.route_ref`` over the router logits ``x @ W_router.T`` and sums
its experts' SwiGLU FFNs with the routing weights (``matmul_ref.moe_ref``,
``draco/models/moe/router.py:81-120``, ``draco/models/moe/expert.py:77-116``);
the reference's GGUF reader rejects such files (``draco/format/gguf.py:616-621``),
so this layer follows its torch MoE modules.

``kv_dtype=np.float16`` rounds each cached key (after RoPE) and value to
float16, the cache dtype of the GPU executor; ``None`` keeps them unrounded
as the reference does with its default float32 cache.  Everything else is
float64.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Sequence

import numpy as np

from oracle import decode_ref, matmul_ref


@dataclass
class ModelSpec:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    eps: float = 1e-5
    theta: float = 10000.0
    tied: bool = False
    experts: int = 0
    top_k: int = 2


def _w(weights: Dict[str, np.ndarray], name: str) -> np.ndarray:
    return np.asarray(weights[name], dtype=np.float64)


def _lin(weights, name, x, bias_name=None):
    y = x @ _w(weights, name).T
    if bias_name is not None and bias_name in weights:
        y = y + _w(weights, bias_name)
    return y


def causal_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """q [L, Hq, D], k / v [L, Hkv, D] (the cached values) -> [L, Hq, D]:
    query t attends to keys 0..t of its kv head h // (Hq / Hkv)."""
    n, hq, d = q.shape
    group = hq // k.shape[1]
    out = np.empty_like(q)
    for h in range(hq):
        kk, vv = k[:, h // group], v[:, h // group]
        s = q[:, h] @ kk.T / np.sqrt(d)
        s = np.where(np.triu(np.ones((n, n), dtype=bool), k=1), -np.inf, s)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ vv
    return out


def llama_forward(weights: Dict[str, np.ndarray], spec: ModelSpec, token_ids: Sequence[int],
                  kv_dtype: Optional[type] = None) -> np.ndarray:
    """Logits [len(token_ids), vocab] of a prompt starting at position 0.

    ``weights`` maps GGUF tensor names (``token_embd.weight``,
    ``blk.N.attn_q.weight`` ..., ``output.weight``) to float arrays of their
    numpy shapes (block-quantized tensors already dequantized); MoE layers
    hold ``blk.N.ffn_gate_inp.weight`` and the 3-D ``blk.N.ffn_{gate,up,down}_exps.weight``."""
    ids = np.asarray(token_ids, dtype=np.int64)
    n = ids.size
    d = spec.hidden // spec.heads
    cos, sin = decode_ref.rope_tables(d, np.arange(n), spec.theta)
    cos, sin = cos.astype(np.float64), sin.astype(np.float64)
    embed = _w(weights, "token_embd.weight")
    h = embed[ids]
    for li in range(spec.layers):
        p = f"blk.{li}."
        x = decode_ref.rms_norm_f64(h, weights[p + "attn_norm.weight"], spec.eps)
        if p + "attn_qkv.weight" in weights:
            qkv = _lin(weights, p + "attn_qkv.weight", x, p + "attn_qkv.bias")
            qd, kvd = spec.heads * d, spec.kv_heads * d
            q, k, v = qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:]
        else:
            q = _lin(weights, p + "attn_q.weight", x, p + "attn_q.bias")
            k = _lin(weights, p + "attn_k.weight", x, p + "attn_k.bias")
            v = _lin(weights, p + "attn_v.weight", x, p + "attn_v.bias")
        q = q.reshape(n, spec.heads, d)
        k = k.reshape(n, spec.kv_heads, d)
        v = v.reshape(n, spec.kv_heads, d)
        q = np.stack([decode_ref.apply_rope(q[t], cos[t], sin[t]) for t in range(n)])
        k = np.stack([decode_ref.apply_rope(k[t], cos[t], sin[t]) for t in range(n)])
        if kv_dtype is not None:
            k = k.astype(kv_dtype).astype(np.float64)
            v = v.astype(kv_dtype).astype(np.float64)
        att = causal_attention(q, k, v).reshape(n, spec.heads * d)
        h = h + _lin(weights, p + "attn_output.weight", att, p + "attn_output.bias")
        x = decode_ref.rms_norm_f64(h, weights[p + "ffn_norm.weight"], spec.eps)
        if p + "ffn_gate_inp.weight" in weights:
            logits = x @ _w(weights, p + "ffn_gate_inp.weight").T
            g, u, dn = (_w(weights, p + f"ffn_{s}_exps.weight") for s in ("gate", "up", "down"))
            h = h + matmul_ref.moe_ref(x, logits, [(g[e], u[e], dn[e]) for e in range(g.shape[0])], spec.top_k)
        else:
            gate = _lin(weights, p + "ffn_gate.weight", x, p + "ffn_gate.bias")
            up = _lin(weights, p + "ffn_up.weight", x, p + "ffn_up.bias")
            h = h + _lin(weights, p + "ffn_down.weight", matmul_ref.silu64(gate) * up, p + "ffn_down.bias")
    x = decode_ref.rms_norm_f64(h, weights["output_norm.weight"], spec.eps)
    head = embed if spec.tied else _w(weights, "output.weight")
    return x @ head.T
