"""Weight-streaming decode step over a Llama-style GGUF layer set.

Counterpart of the reference executor's per-token projection sequence:
``forward_step`` / ``forward_batch_decode`` run, per layer, ``_qkv`` (3x
``_linear``), ``_o_proj`` and ``_mlp`` (gate, up, SwiGLU, down), then the
final ``lm_head`` ``_linear`` (``draco/runtime/cpu/executor.py:208-277,
290-396``).  Here a layer is four fused dequant-GEMV launches over the packed
GGUF blocks -- q/k/v in one launch, o with the residual add, gate/up with the
SwiGLU product, down with the residual add -- plus one for the lm_head, and
the whole step can be captured into one HIP graph.  The projection inputs are
bfloat16 (each launch writes the bf16 copy its consumer reads); the residual
stream and the logits are float32.

Two forms of the step:

* projections only (``attention=None``): the attention output fed to
  ``o_proj`` is the q projection itself and there are no norms, so a step
  streams exactly the layer set's weight bytes (the headline workload);
* the full decode step (``attention=AttentionShape(...)``): per layer
  RMSNorm -> q/k/v -> RoPE + KV-cache append + attention -> o_proj (+ residual)
  -> RMSNorm -> gate/up SwiGLU -> down (+ residual), then the final RMSNorm and
  the lm_head, as ``forward_step`` runs it
  (``draco/runtime/cpu/executor.py:290-342``); every step appends one token
  per sequence to the float16 caches and advances the device positions.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

from dracort_amd.exceptions import KVCacheError
from dracort_amd.format.gguf import GGML_TYPE_Q4_K, GGML_TYPE_Q6_K, tensor_bytes
from dracort_amd.kernels.dense import get_rows
from dracort_amd.kernels.glue import DecodeAttentionWorkspace, decode_attention, rms_norm, rope_tables
from dracort_amd.kernels.gguf import (
    gguf_gemv,
    gguf_gemv_multi,
    gguf_gemv_multi_rmsnorm,
    gguf_gemv_residual,
    gemv_residual_workspace_bytes,
    gguf_gemv_swiglu,
    gguf_gemv_swiglu_rmsnorm,
)
from dracort_amd.quantization.gguf import GGUFQuantizedWeight
from dracort_amd.quantization.quantize import quantize

PROJ = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass
class LlamaShape:
    hidden: int = 4096
    inter: int = 14336
    kv_dim: int = 1024
    vocab: int = 128256
    n_layers: int = 32

    def proj_shape(self, name: str):
        h, i, kv = self.hidden, self.inter, self.kv_dim
        return {"q": (h, h), "k": (kv, h), "v": (kv, h), "o": (h, h), "gate": (i, h), "up": (i, h),
                "down": (h, i)}[name]


# Q4_K_M assignment used by the layer-set workload: Q4_K for attention and
# gate/up, Q6_K for down and lm_head.
Q4_K_M_TYPES = {"q": GGML_TYPE_Q4_K, "k": GGML_TYPE_Q4_K, "v": GGML_TYPE_Q4_K, "o": GGML_TYPE_Q4_K,
                "gate": GGML_TYPE_Q4_K, "up": GGML_TYPE_Q4_K, "down": GGML_TYPE_Q6_K}


@dataclass
class AttentionShape:
    """Llama-3-8B attention: 32 query heads, 8 kv heads of 128, RoPE theta 500000."""

    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    max_positions: int = 8192


@dataclass
class LayerSet:
    shape: LlamaShape
    layers: List[Dict[str, GGUFQuantizedWeight]] = field(default_factory=list)
    lm_head: Optional[GGUFQuantizedWeight] = None
    # float32 RMSNorm weights per layer ("attn", "ffn") and the final one
    norms: List[Dict[str, torch.Tensor]] = field(default_factory=list)
    output_norm: Optional[torch.Tensor] = None
    # token embedding table (raw bytes on the device, its ggml type and [vocab, hidden] shape), if any
    embed: Optional[Tuple[torch.Tensor, int, Tuple[int, int]]] = None

    @property
    def weight_bytes(self) -> int:
        total = sum(w.nbytes for layer in self.layers for w in layer.values())
        return total + (self.lm_head.nbytes if self.lm_head is not None else 0)


def synthetic_weight(n: int, k: int, ggml_type: int, gen: torch.Generator, device) -> GGUFQuantizedWeight:
    """N(0, 0.02) weight with 1 % of its rows (seeded) scaled x4, quantized on the device."""
    w = torch.randn((n, k), generator=gen, device=device, dtype=torch.float32).mul_(0.02)
    rows = torch.randperm(n, generator=gen, device=device)[: max(1, n // 100)]
    w[rows] *= 4.0
    q = quantize(w, ggml_type)
    del w
    return GGUFQuantizedWeight(q, ggml_type, (n, k))


def synthetic_layer_set(shape: LlamaShape, seed: int = 0, device="cuda", types=None,
                        lm_head_type: int = GGML_TYPE_Q6_K) -> LayerSet:
    types = dict(Q4_K_M_TYPES if types is None else types)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    ls = LayerSet(shape)
    for _ in range(shape.n_layers):
        layer = {}
        for name in PROJ:
            n, k = shape.proj_shape(name)
            layer[name] = synthetic_weight(n, k, types[name], gen, device)
        ls.layers.append(layer)
    ls.lm_head = synthetic_weight(shape.vocab, shape.hidden, lm_head_type, gen, device)
    for _ in range(shape.n_layers):
        ls.norms.append({p: 1.0 + 0.1 * torch.randn(shape.hidden, generator=gen, device=device)
                         for p in ("attn", "ffn")})
    ls.output_norm = 1.0 + 0.1 * torch.randn(shape.hidden, generator=gen, device=device)
    return ls


def layer_set_from_gguf(reader, device="cuda", max_positions: Optional[int] = None):
    """(LayerSet, AttentionShape) of a dense llama-family GGUF file for the
    fused decode step: the tensor names and metadata the reference's
    ``_build_index`` / ``_build_metadata`` read (``draco/format/gguf.py:604-772``)
    and ``CPUExecutorConfig.from_metadata`` consumes
    (``draco/runtime/cpu/executor.py:108-129``), every projection uploaded in
    its packed layout, the token embedding table kept for the gather.  The
    step's fused launches need block-quantized q/k/v/o/gate/up/down and
    lm_head with whole blocks per row, gate and up of one type, no biases and
    no experts; other files run on :class:`GPUExecutionBackend`."""
    from dracort_amd.format.gguf import BLOCK_LAYOUTS, base_type
    from dracort_amd.runtime.executor import gguf_executor_config
    from dracort_amd.weights.upload import upload_gguf

    cfg = gguf_executor_config(reader)
    if cfg.num_experts or cfg.qkv_fused or cfg.attention_bias or cfg.mlp_bias:
        raise ValueError("the fused decode step takes dense models with separate, bias-free q/k/v projections")
    hd = cfg.head_dim
    names = ["token_embd.weight", "output_norm.weight"] + ([] if cfg.tie_word_embeddings else ["output.weight"])
    gg = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate", "up": "ffn_up",
          "down": "ffn_down"}
    for i in range(cfg.num_hidden_layers):
        names += [f"blk.{i}.{gg[p]}.weight" for p in PROJ] + [f"blk.{i}.attn_norm.weight", f"blk.{i}.ffn_norm.weight"]
    up = upload_gguf(reader, names, device=device)

    def block(name):
        w = up[name]
        if not isinstance(w, GGUFQuantizedWeight):
            raise ValueError(f"'{name}' is not a block-quantized tensor with whole blocks per row")
        return w

    def f32(name):
        t = up[name]
        if not isinstance(t, torch.Tensor) or not t.is_floating_point():
            raise ValueError(f"'{name}' must be a float tensor")
        return t.to(torch.float32).reshape(-1).contiguous()

    inter = cfg.intermediate_size or reader.tensor("blk.0.ffn_gate.weight").shape[0]
    shape = LlamaShape(hidden=cfg.hidden_size, inter=inter, kv_dim=cfg.num_key_value_heads * hd,
                       vocab=cfg.vocab_size, n_layers=cfg.num_hidden_layers)
    ls = LayerSet(shape)
    for i in range(cfg.num_hidden_layers):
        layer = {p: block(f"blk.{i}.{gg[p]}.weight") for p in PROJ}
        if layer["gate"].ggml_type != layer["up"].ggml_type:
            raise ValueError(f"layer {i}: gate and up projections of different types")
        for p in PROJ:
            if tuple(layer[p].shape) != shape.proj_shape(p):
                raise ValueError(f"layer {i} {p}: shape {layer[p].shape}, expected {shape.proj_shape(p)}")
        ls.layers.append(layer)
        ls.norms.append({"attn": f32(f"blk.{i}.attn_norm.weight"), "ffn": f32(f"blk.{i}.ffn_norm.weight")})
    ls.output_norm = f32("output_norm.weight")
    et = reader.tensor("token_embd.weight")
    e = up["token_embd.weight"]
    edata = e.data if isinstance(e, GGUFQuantizedWeight) else e.reshape(-1).view(torch.uint8)
    ekind = e.ggml_type if isinstance(e, GGUFQuantizedWeight) else et.info.ggml_type
    ls.embed = (edata, ekind, tuple(et.shape))
    if cfg.tie_word_embeddings:
        if not isinstance(e, GGUFQuantizedWeight) or base_type(e.ggml_type) not in BLOCK_LAYOUTS:
            raise ValueError("tied embeddings must be block-quantized for the fused decode step's lm_head")
        ls.lm_head = e
    else:
        ls.lm_head = block("output.weight")
    attn = AttentionShape(n_heads=cfg.num_attention_heads, n_kv_heads=cfg.num_key_value_heads, head_dim=hd,
                          rope_theta=cfg.rope_theta, rms_eps=cfg.rms_norm_eps,
                          max_positions=int(max_positions or cfg.max_position_embeddings))
    return ls, attn


def layer_set_bytes(shape: LlamaShape, types=None, lm_head_type: int = GGML_TYPE_Q6_K) -> int:
    types = dict(Q4_K_M_TYPES if types is None else types)
    per_layer = sum(tensor_bytes(types[p], shape.proj_shape(p)) for p in PROJ)
    return shape.n_layers * per_layer + tensor_bytes(lm_head_type, (shape.vocab, shape.hidden))


class DecodeStep:
    """Preallocated buffers + the decode chain for a batch of `m` tokens (one
    per sequence); ``attention`` selects the full step (see the module doc),
    with ``start_position`` tokens already cached per sequence.

    The full step keeps a host-side count of the position it will write next
    (the device positions advance by one per step, eager or replayed): a step
    that would write position ``max_positions`` raises ``KVCacheError`` before
    anything is enqueued."""

    def __init__(self, ls: LayerSet, m: int = 1, device="cuda", attention: Optional[AttentionShape] = None,
                 start_position: int = 0) -> None:
        s = ls.shape
        self.ls, self.m, self.attn = ls, m, attention
        f32 = dict(dtype=torch.float32, device=device)
        b16 = dict(dtype=torch.bfloat16, device=device)
        gen = torch.Generator(device=device).manual_seed(1234)
        self.x_in = torch.randn((m, s.hidden), generator=gen, **f32).to(torch.bfloat16)
        self.h = torch.empty((m, s.hidden), **f32)
        self.h_bf16 = torch.empty((m, s.hidden), **b16)
        self.q = torch.empty((m, s.hidden), **b16)
        self.k = torch.empty((m, s.kv_dim), **b16)
        self.v = torch.empty((m, s.kv_dim), **b16)
        self.s = torch.empty((m, s.inter), **b16)
        self.logits = torch.empty((m, s.vocab), **f32)
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        # split-K room of the residual projections (the down projection at
        # several tokens); one buffer, the launches run one after another
        ws_bytes = max([gemv_residual_workspace_bytes(w.ggml_type, m, w.shape[0], w.shape[1])
                        for layer in ls.layers for w in (layer["o"], layer["down"])] + [0])
        self.gemv_ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
        if attention is not None:
            a = attention
            if a.n_heads * a.head_dim != s.hidden or a.n_kv_heads * a.head_dim != s.kv_dim:
                raise ValueError("attention heads do not match the projection shapes")
            if not ls.norms or ls.output_norm is None:
                raise ValueError("the full decode step needs the layer set's RMSNorm weights")
            if not 0 <= start_position < a.max_positions:
                raise ValueError(f"start_position must be in [0, {a.max_positions})")
            cache = (m, a.n_kv_heads, a.max_positions, a.head_dim)
            self.k_cache = [torch.zeros(cache, dtype=torch.float16, device=device) for _ in ls.layers]
            self.v_cache = [torch.zeros(cache, dtype=torch.float16, device=device) for _ in ls.layers]
            self.positions = torch.full((m,), start_position, dtype=torch.int32, device=device)
            self.next_position = start_position
            self.rope = rope_tables(a.head_dim, a.max_positions, a.rope_theta, device)
            self.ws = DecodeAttentionWorkspace(m, a.n_heads, a.n_kv_heads, a.head_dim, a.max_positions, device)
            self.qf = torch.empty((m, s.hidden), **f32)
            self.kf = torch.empty((m, s.kv_dim), **f32)
            self.vf = torch.empty((m, s.kv_dim), **f32)
            self.xn = torch.empty((m, s.hidden), **b16)
            self.att = torch.empty((m, s.hidden), **b16)
        # token input through the embedding gather (set_tokens); otherwise x_in
        self.ids = torch.zeros((m,), dtype=torch.int32, device=device) if ls.embed is not None else None
        self.use_tokens = False

    def set_tokens(self, ids) -> None:
        """The next step's input tokens (one per sequence): their embedding rows
        replace x_in.  The ids buffer is updated in place, so a captured graph
        picks them up on its next replay."""
        if self.ids is None:
            raise ValueError("the layer set carries no embedding table")
        t = torch.as_tensor(ids, dtype=torch.int32).reshape(-1)
        if t.numel() != self.m:
            raise ValueError(f"need {self.m} token ids, got {t.numel()}")
        vocab = self.ls.embed[2][0]
        if int(t.min()) < 0 or int(t.max()) >= vocab:
            raise ValueError(f"token ids must be in [0, {vocab})")
        self.ids.copy_(t.to(self.ids.device))
        self.use_tokens = True

    def _input(self) -> None:
        if self.use_tokens:
            table, gt, shp = self.ls.embed
            get_rows(table, gt, shp, self.ids, out=self.h)
        else:
            self.h.copy_(self.x_in)

    def run(self) -> torch.Tensor:
        if self.attn is not None:
            return self._run_full()
        s = self.ls.shape
        self.h.copy_(self.x_in)
        self.h_bf16.copy_(self.x_in)
        for layer in self.ls.layers:
            q, k, v, o = layer["q"], layer["k"], layer["v"], layer["o"]
            if q.ggml_type == k.ggml_type == v.ggml_type:
                gguf_gemv_multi(self.h_bf16, [(q.data, q.shape[0]), (k.data, k.shape[0]), (v.data, v.shape[0])],
                                q.ggml_type, s.hidden, [None, None, None], [self.q, self.k, self.v])
            else:
                for w, out in ((q, self.q), (k, self.k), (v, self.v)):
                    gguf_gemv_multi(self.h_bf16, [(w.data, w.shape[0])], w.ggml_type, s.hidden, [None], [out])
            gguf_gemv_residual(self.q, o.data, o.ggml_type, o.shape, self.h, self.h_bf16, workspace=self.gemv_ws)
            g, u, d = layer["gate"], layer["up"], layer["down"]
            gguf_gemv_swiglu(self.h_bf16, g.data, u.data, g.ggml_type, g.shape, out_bf16=self.s)
            gguf_gemv_residual(self.s, d.data, d.ggml_type, d.shape, self.h, self.h_bf16, workspace=self.gemv_ws)
        w = self.ls.lm_head
        gguf_gemv(self.h_bf16, w.data, w.ggml_type, w.shape, out=self.logits)
        return self.logits

    def _claim_position(self) -> None:
        if self.next_position >= self.attn.max_positions:
            raise KVCacheError(f"KV cache full: position {self.next_position} is past max_positions "
                               f"{self.attn.max_positions}")
        self.next_position += 1

    def _run_full(self) -> torch.Tensor:
        s, a = self.ls.shape, self.attn
        self._claim_position()
        self._input()
        for li, layer in enumerate(self.ls.layers):
            norms = self.ls.norms[li]
            q, k, v, o = layer["q"], layer["k"], layer["v"], layer["o"]
            if q.ggml_type == k.ggml_type == v.ggml_type:
                # the attention norm runs in the q/k/v launch's prologue
                gguf_gemv_multi_rmsnorm(self.h, norms["attn"], a.rms_eps, self.xn,
                                        [(q.data, q.shape[0]), (k.data, k.shape[0]), (v.data, v.shape[0])],
                                        q.ggml_type, s.hidden, [self.qf, self.kf, self.vf])
            else:
                rms_norm(self.h, norms["attn"], a.rms_eps, out_bf16=self.xn)
                for w, out in ((q, self.qf), (k, self.kf), (v, self.vf)):
                    gguf_gemv_multi(self.xn, [(w.data, w.shape[0])], w.ggml_type, s.hidden, [out])
            decode_attention(self.qf, self.kf, self.vf, self.k_cache[li], self.v_cache[li], self.positions,
                             a.n_heads, a.n_kv_heads, rope=self.rope, out=self.att, workspace=self.ws)
            gguf_gemv_residual(self.att, o.data, o.ggml_type, o.shape, self.h, workspace=self.gemv_ws)
            g, u, d = layer["gate"], layer["up"], layer["down"]
            gguf_gemv_swiglu_rmsnorm(self.h, norms["ffn"], a.rms_eps, self.xn, g.data, u.data, g.ggml_type, g.shape,
                                     out_bf16=self.s)
            gguf_gemv_residual(self.s, d.data, d.ggml_type, d.shape, self.h, workspace=self.gemv_ws)
        w = self.ls.lm_head
        gguf_gemv_multi_rmsnorm(self.h, self.ls.output_norm, a.rms_eps, self.xn, [(w.data, w.shape[0])],
                                w.ggml_type, s.hidden, [self.logits])
        self.positions.add_(1)
        return self.logits

    def capture(self) -> None:
        """Capture one step into a HIP graph (replay with ``replay``).

        One eager step runs first (allocator and library warm-up).  For the
        full step its only lasting effect is undone: the device positions and
        the host count are put back, so the first replay writes the same
        position again (overwriting the warm-up's cache entry)."""
        saved = self.positions.clone() if self.attn is not None else None
        saved_next = self.next_position if self.attn is not None else None
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.run()  # warm the allocator / library outside capture
            if saved is not None:
                self.positions.copy_(saved)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.run()
        if saved_next is not None:
            self.next_position = saved_next  # capturing enqueues nothing
        self.graph = g

    def replay(self) -> torch.Tensor:
        assert self.graph is not None
        if self.attn is not None:
            self._claim_position()
        self.graph.replay()
        return self.logits
