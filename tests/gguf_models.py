"""Small GGUF model files for the executor tests, written with tests/gguf_writer.py.

``write_llama`` writes a llama-family file (dense or MoE) whose projections are
block-quantized with this package's quantizers, and returns the oracle's view
of it: every tensor as float64 (block tensors dequantized by the oracle from
the very bytes written), ready for ``oracle.model_ref.llama_forward``.
``write_reference_tiny`` restates the reference's own end-to-end fixture
``_tiny_gguf_model`` (``tests/format/test_gguf.py:644-700``: qwen2, hidden 16,
2 layers, 4 heads of 4, 2 kv heads, intermediate 32, vocabulary 32, Q8_0
``ffn_gate`` / ``ffn_up`` of shape [32, 16] whose blocks run across rows,
float32 elsewhere, weights N(0, 1) x 0.05 from ``default_rng(0)`` in the
fixture's order) and returns both the oracle's view and the unquantized
weights its independent reference uses."""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np
import torch

from dracort_amd.quantization import quantize
from oracle import encoders, gguf_ref
from tests.gguf_writer import write_gguf


def _quantized(arr: np.ndarray, qtype: int):
    """(payload bytes, oracle float64 dequantization) of a float32 array."""
    flat = arr.reshape(-1, arr.shape[-1]).astype(np.float32)
    blocks = quantize(torch.from_numpy(flat), qtype).numpy()
    deq = gguf_ref.dequantize(qtype & ~0x100, blocks, flat.size, ggml_order=bool(qtype & 0x100))
    return blocks.tobytes(), deq.reshape(arr.shape).astype(np.float64)


def write_llama(path: str, *, hidden=256, layers=2, heads=4, kv_heads=2, inter=512, vocab=384, seed=0,
                types: Optional[Dict[str, int]] = None, embed_type=1, out_type: Optional[int] = 8,
                experts=0, top_k=2, expert_type=12, arch="llama", eps=1e-5, theta=10000.0, context=256,
                bias=False):
    """Returns the oracle's float64 weights by GGUF name.  types: per projection
    ("q", "k", "v", "o", "gate", "up", "down") ggml type; embed_type 0 (F32),
    1 (F16) or a block type; out_type None ties the output to the embeddings."""
    types = dict({"q": 12, "k": 12, "v": 14, "o": 12, "gate": 12, "up": 12, "down": 14}, **(types or {}))
    rng = np.random.default_rng(seed)
    d = hidden // heads
    tensors, ref = [], {}

    def add_float(name, arr, ttype=0):
        arr = arr.astype(np.float32)
        if ttype == 1:
            a16 = arr.astype(np.float16)
            tensors.append((name, arr.shape, 1, a16.tobytes()))
            ref[name] = a16.astype(np.float64)
        else:
            tensors.append((name, arr.shape, 0, arr.tobytes()))
            ref[name] = arr.astype(np.float64)

    def add_weight(name, shape, ttype, scale=0.02):
        arr = (rng.standard_normal(shape) * scale).astype(np.float32)
        if ttype in (0, 1):
            add_float(name, arr, ttype)
            return
        payload, deq = _quantized(arr, ttype)
        tensors.append((name, shape, ttype, payload))
        ref[name] = deq

    add_weight("token_embd.weight", (vocab, hidden), embed_type, scale=1.0)
    gg = {"q": ("attn_q", (heads * d, hidden)), "k": ("attn_k", (kv_heads * d, hidden)),
          "v": ("attn_v", (kv_heads * d, hidden)), "o": ("attn_output", (hidden, heads * d)),
          "gate": ("ffn_gate", (inter, hidden)), "up": ("ffn_up", (inter, hidden)), "down": ("ffn_down", (hidden, inter))}
    for i in range(layers):
        p = f"blk.{i}."
        add_float(p + "attn_norm.weight", 1 + 0.1 * rng.standard_normal(hidden))
        add_float(p + "ffn_norm.weight", 1 + 0.1 * rng.standard_normal(hidden))
        for key in ("q", "k", "v", "o"):
            gname, shape = gg[key]
            add_weight(p + gname + ".weight", shape, types[key])
            if bias and key in ("q", "k", "v"):
                add_float(p + gname + ".bias", 0.1 * rng.standard_normal(shape[0]))
        if experts:
            add_float(p + "ffn_gate_inp.weight", rng.standard_normal((experts, hidden)) * 0.1)
            for s, shape in (("gate", (experts, inter, hidden)), ("up", (experts, inter, hidden)),
                             ("down", (experts, hidden, inter))):
                add_weight(p + f"ffn_{s}_exps.weight", shape, expert_type)
        else:
            for key in ("gate", "up", "down"):
                gname, shape = gg[key]
                add_weight(p + gname + ".weight", shape, types[key])
    add_float("output_norm.weight", 1 + 0.1 * rng.standard_normal(hidden))
    if out_type is not None:
        add_weight("output.weight", (vocab, hidden), out_type, scale=0.05)
    meta = [("general.architecture", "str", arch), (f"{arch}.embedding_length", "u32", hidden),
            (f"{arch}.block_count", "u32", layers), (f"{arch}.feed_forward_length", "u32", inter),
            (f"{arch}.attention.head_count", "u32", heads), (f"{arch}.attention.head_count_kv", "u32", kv_heads),
            (f"{arch}.vocab_size", "u32", vocab), (f"{arch}.context_length", "u32", context),
            (f"{arch}.attention.layer_norm_rms_epsilon", "f32", eps), (f"{arch}.rope.freq_base", "f32", theta)]
    if experts:
        meta += [(f"{arch}.expert_count", "u32", experts), (f"{arch}.expert_used_count", "u32", top_k)]
    write_gguf(path, meta, tensors)
    return ref


def write_reference_tiny(path: str):
    """(oracle float64 weights, the fixture's unquantized float64 weights)."""
    hidden, layers, heads, kv_heads, inter, vocab = 16, 2, 4, 2, 32, 32
    d = hidden // heads
    rng = np.random.default_rng(0)
    tensors, ref, orig = [], {}, {}

    def add(name, shape, quant=False):
        arr = (rng.normal(size=shape) * 0.05).astype(np.float32)
        orig[name] = arr.astype(np.float64)
        if quant:
            payload = encoders.enc_q8_0(arr.reshape(-1))
            tensors.append((name, shape, 8, payload))
            ref[name] = gguf_ref.dequantize(8, np.frombuffer(payload, np.uint8), arr.size).reshape(shape) \
                .astype(np.float64)
        else:
            tensors.append((name, shape, 0, arr.tobytes()))
            ref[name] = arr.astype(np.float64)

    add("token_embd.weight", (vocab, hidden))
    for i in range(layers):
        p = f"blk.{i}."
        add(p + "attn_norm.weight", (hidden,))
        add(p + "attn_q.weight", (heads * d, hidden))
        add(p + "attn_k.weight", (kv_heads * d, hidden))
        add(p + "attn_v.weight", (kv_heads * d, hidden))
        add(p + "attn_output.weight", (hidden, heads * d))
        add(p + "ffn_norm.weight", (hidden,))
        add(p + "ffn_gate.weight", (inter, hidden), quant=True)
        add(p + "ffn_up.weight", (inter, hidden), quant=True)
        add(p + "ffn_down.weight", (hidden, inter))
    add("output_norm.weight", (hidden,))
    add("output.weight", (vocab, hidden))
    meta = [("general.architecture", "str", "qwen2"), ("qwen2.embedding_length", "u32", hidden),
            ("qwen2.block_count", "u32", layers), ("qwen2.feed_forward_length", "u32", inter),
            ("qwen2.attention.head_count", "u32", heads), ("qwen2.attention.head_count_kv", "u32", kv_heads),
            ("qwen2.vocab_size", "u32", vocab), ("qwen2.context_length", "u32", 64),
            ("qwen2.attention.layer_norm_rms_epsilon", "f32", 1e-6)]
    write_gguf(path, meta, tensors)
    return ref, orig
