"""GPU execution backend for GGUF models: a ``.gguf`` file decodes tokens on
the MI355X.

Counterpart of the reference's ``CPUExecutionBackend`` built from a
``GGUFReader`` (``draco/runtime/cpu/executor.py:131-396``, metadata from
``GGUFReader._build_index`` / ``_build_metadata``,
``draco/format/gguf.py:604-772``) for the llama family the reference's GGUF
path accepts (``_ARCH_FAMILY``, ``draco/format/gguf.py:106-118``: llama,
qwen2, qwen3, mistral, phi3, yi, starcoder2 -- RMSNorm, RoPE, gated MLP,
separate or fused q/k/v, optional attention / MLP biases, tied or separate
output head) and, beyond the reference, which rejects them
(``draco/format/gguf.py:616-621``), sparse-MoE GGUF files: per layer an
``ffn_gate_inp`` router linear and 3-D ``ffn_{gate,up,down}_exps`` expert
stacks, routed top-k with softmax over the selected logits.

Every weight stays in HBM in its file layout: block-quantized tensors feed
the fused dequant-GEMV kernels; float tensors (F32 / F16 / BF16) the dense
linear kernel; a block tensor whose blocks run across rows (K not a multiple
of the block size) is dequantized once, bit-exactly, into a float32 copy (the
reference caches every weight as float32 the same way,
``draco/format/gguf.py:827-834``).  Activations between launches are float32,
as in the reference's numpy chain; the KV cache is float16
``[max_num_seqs, kv heads, max_positions, head_dim]`` per layer, position p of
a sequence holding its token p.

A prompt is run one token at a time through the decode kernels (the causal
attention over the prompt is exactly the per-token decode attention over the
growing cache).  ``forward_batch_decode`` batches the projections of up to 16
sequences per launch and runs the attention per sequence, as the reference
does.  The gpt2 family (LayerNorm, learned positions, GELU) is not part of
this path and raises.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Union

import numpy as np
import torch

from dracort_amd.exceptions import CPUError, DracoFormatError, KVCacheError
from dracort_amd.format.gguf import BLOCK_LAYOUTS, base_type, tensor_bytes
from dracort_amd.format.gguf_file import FLOAT_TYPES, GGUFFile
from dracort_amd.kernels.dense import dense_linear, get_rows, swiglu
from dracort_amd.kernels.glue import DecodeAttentionWorkspace, decode_attention, rms_norm, rope_tables
from dracort_amd.kernels.gguf import (
    GEMV_MAX_M,
    gguf_dequantize,
    gguf_gemv_multi,
    gguf_gemv_residual,
    gguf_gemv_swiglu,
    gguf_linear,
    gguf_moe,
)
from dracort_amd.weights.upload import upload_gguf

# the reference's llama-family GGUF architectures (draco/format/gguf.py:106-118)
LLAMA_FAMILY = ("llama", "mistral", "phi3", "qwen2", "qwen3", "starcoder2", "yi")


@dataclass
class GPUExecutorConfig:
    """The llama-family fields of the reference's ``CPUExecutorConfig``
    (``draco/runtime/cpu/executor.py:82-129``) plus the MoE sizes."""

    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    intermediate_size: int = 0
    rope_theta: float = 10000.0
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-5
    tie_word_embeddings: bool = False
    qkv_fused: bool = False
    attention_bias: bool = False
    mlp_bias: bool = False
    num_experts: int = 0
    num_experts_per_tok: int = 0
    architecture: str = "llama"

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


def gguf_executor_config(reader: GGUFFile) -> GPUExecutorConfig:
    """Executor configuration from a GGUF file's metadata, as the reference's
    ``_build_metadata`` reads it for the llama family
    (``draco/format/gguf.py:664-760``)."""
    meta = reader.metadata
    arch = meta.get("general.architecture", "")
    if arch not in LLAMA_FAMILY:
        raise DracoFormatError(
            f"GGUF architecture '{arch}' is not supported by the GPU executor. Supported: {list(LLAMA_FAMILY)} "
            f"(llama-family models with standard blk.* tensor names)."
        )
    p = arch + "."
    names = set(reader.tensor_names())

    def get(key, cast, default=None):
        v = meta.get(p + key)
        if v is None:
            return default
        try:
            return cast(v)
        except (TypeError, ValueError):
            return default

    hidden = get("embedding_length", int)
    layers = get("block_count", int)
    heads = get("attention.head_count", int)
    kv_heads = get("attention.head_count_kv", int) or heads
    vocab = get("vocab_size", int)
    if vocab is None and "token_embd.weight" in names:
        vocab = reader.tensor("token_embd.weight").shape[0]
    if None in (hidden, layers, heads, vocab):
        raise DracoFormatError(
            f"GGUF '{reader.path}' is missing required architecture metadata "
            f"(embedding_length / block_count / attention.head_count / vocab_size)."
        )
    key_len = get("attention.key_length", int)
    if key_len is not None and key_len != hidden // heads:
        raise DracoFormatError(
            f"GGUF '{reader.path}' uses a non-standard key_length {key_len} (head_dim={hidden // heads}); the "
            f"executor requires head_dim == hidden_size // head_count."
        )
    rms_eps = get("attention.layer_norm_rms_epsilon", float) or get("attention.layer_norm_epsilon", float) or 1e-5
    has_output = "output.weight" in names
    tie = meta.get(p + "tie_embeddings")
    inter = get("feed_forward_length", int) or 0
    experts = get("expert_count", int) or 0
    if experts and "blk.0.ffn_gate_exps.weight" not in names:
        experts = 0
    return GPUExecutorConfig(
        hidden_size=hidden, num_hidden_layers=layers, num_attention_heads=heads, num_key_value_heads=kv_heads,
        vocab_size=vocab, intermediate_size=inter, rope_theta=get("rope.freq_base", float, 10000.0) or 10000.0,
        max_position_embeddings=get("context_length", int) or 4096, rms_norm_eps=float(rms_eps),
        tie_word_embeddings=bool(tie) if tie is not None else not has_output,
        qkv_fused="blk.0.attn_qkv.weight" in names,
        attention_bias="blk.0.attn_q.bias" in names or "blk.0.attn_qkv.bias" in names,
        mlp_bias="blk.0.ffn_gate.bias" in names or "blk.0.ffn_up.bias" in names,
        num_experts=experts, num_experts_per_tok=(get("expert_used_count", int) or 2) if experts else 0,
        architecture=arch,
    )


@dataclass
class DeviceWeight:
    """A GGUF tensor in HBM as the kernels take it.

    kind ``block``: packed blocks, whole blocks per row (fused GEMV / GEMM);
    ``float``: an F32 / F16 / BF16 tensor (dense kernel; ``data`` its bytes);
    ``flat``: packed blocks running across rows, used through ``dense``, its
    bit-exact float32 dequantization."""

    name: str
    ggml_type: int
    shape: tuple
    data: torch.Tensor
    kind: str
    dense: Optional[torch.Tensor] = None

    @property
    def n(self) -> int:
        return int(self.shape[0])

    @property
    def k(self) -> int:
        return int(self.shape[-1])


def _device_weight(name: str, t, up) -> DeviceWeight:
    ttype = t.info.ggml_type
    shape = tuple(t.shape)
    if ttype in FLOAT_TYPES:
        if ttype == 28:
            raise DracoFormatError(f"GGUF tensor '{name}' is F64, which the GPU kernels do not read")
        data = up if up.dtype == torch.uint8 else up.reshape(-1).view(torch.uint8)
        return DeviceWeight(name, ttype, shape, data, "float")
    raw = up.data if hasattr(up, "data") and not isinstance(up, torch.Tensor) else up
    if base_type(t.kernel_type) not in BLOCK_LAYOUTS:
        raise DracoFormatError(f"GGUF tensor '{name}' has unsupported ggml type {ttype}")
    qk = BLOCK_LAYOUTS[base_type(t.kernel_type)][0]
    if len(shape) == 2 and shape[1] % qk == 0:
        return DeviceWeight(name, t.kernel_type, shape, raw, "block")
    if len(shape) == 2:
        dense = gguf_dequantize(raw, t.kernel_type, shape)
        return DeviceWeight(name, t.kernel_type, shape, raw, "flat", dense=dense)
    return DeviceWeight(name, t.kernel_type, shape, raw, "stack")  # 3-D expert stack


@dataclass
class _Layer:
    attn_norm: torch.Tensor
    ffn_norm: torch.Tensor
    q: Optional[DeviceWeight] = None
    k: Optional[DeviceWeight] = None
    v: Optional[DeviceWeight] = None
    qkv: Optional[DeviceWeight] = None
    o: Optional[DeviceWeight] = None
    gate: Optional[DeviceWeight] = None
    up: Optional[DeviceWeight] = None
    down: Optional[DeviceWeight] = None
    router: Optional[DeviceWeight] = None
    experts: Optional[Dict[str, List[torch.Tensor]]] = None
    expert_type: int = 0
    bias: Dict[str, torch.Tensor] = field(default_factory=dict)


class GPUExecutionBackend:
    """Runs a llama-family (dense or MoE) GGUF model's decode steps on one GPU.

    Interface of the reference's ``CPUExecutionBackend``: ``new_sequence``,
    ``end_sequence``, ``truncate_sequence``, ``forward_step(seq_id, token_ids,
    start_position, return_all_positions=False)`` and
    ``forward_batch_decode(seq_ids, token_ids, positions)`` returning float32
    numpy logits, ``generate_greedy``.  ``start_position`` must equal the
    number of tokens the sequence has cached (the reference appends at the
    cache's end whatever it is told; here the cache is indexed by position)."""

    def __init__(self, reader: Union[GGUFFile, str], max_num_seqs: int = 1, max_positions: Optional[int] = None,
                 device: Union[str, torch.device] = "cuda", field_order: str = "reference") -> None:
        self._own_reader = isinstance(reader, str)
        self.reader = GGUFFile(reader, field_order=field_order) if isinstance(reader, str) else reader
        self.config = cfg = gguf_executor_config(self.reader)
        self.device = torch.device(device)
        if self.device.type != "cuda" or not torch.cuda.is_available():
            raise CPUError("the GPU execution backend needs a GPU (there is no CPU fallback)")
        self.max_positions = int(max_positions or cfg.max_position_embeddings)
        self.max_num_seqs = int(max_num_seqs)
        hd = cfg.head_dim
        if cfg.num_attention_heads * hd != cfg.hidden_size:
            raise DracoFormatError("hidden_size must be num_attention_heads * head_dim")
        self._load_weights()
        dev = dict(device=self.device)
        cache = (self.max_num_seqs, cfg.num_key_value_heads, self.max_positions, hd)
        self.k_cache = [torch.zeros(cache, dtype=torch.float16, **dev) for _ in range(cfg.num_hidden_layers)]
        self.v_cache = [torch.zeros(cache, dtype=torch.float16, **dev) for _ in range(cfg.num_hidden_layers)]
        self.rope = rope_tables(hd, self.max_positions, cfg.rope_theta, self.device)
        self.attn_ws = DecodeAttentionWorkspace(1, cfg.num_attention_heads, cfg.num_key_value_heads, hd,
                                                self.max_positions, self.device)
        self._slots: Dict[int, int] = {}
        self._length: Dict[int, int] = {}
        self._next_seq_id = 0

    # -- weights ---------------------------------------------------------
    def _load_weights(self) -> None:
        cfg, r = self.config, self.reader
        names = r.tensor_names()
        up = upload_gguf(r, names, device=self.device)
        w = {n: _device_weight(n, r.tensor(n), up[n]) for n in names}

        def need(name):
            if name not in w:
                raise CPUError(f"Could not find weight tensor '{name}' in '{r.path}'.")
            return w[name]

        def norm(name):
            t = need(name)
            if t.kind != "float":
                raise DracoFormatError(f"norm weight '{name}' must be a float tensor")
            return _as_f32(t)

        self.embed = need("token_embd.weight")
        self.output_norm = norm("output_norm.weight")
        self.lm_head = self.embed if cfg.tie_word_embeddings else need("output.weight")
        self.layers: List[_Layer] = []
        for i in range(cfg.num_hidden_layers):
            p = f"blk.{i}."
            L = _Layer(attn_norm=norm(p + "attn_norm.weight"), ffn_norm=norm(p + "ffn_norm.weight"))
            if cfg.qkv_fused:
                L.qkv = need(p + "attn_qkv.weight")
            else:
                L.q, L.k, L.v = need(p + "attn_q.weight"), need(p + "attn_k.weight"), need(p + "attn_v.weight")
            L.o = need(p + "attn_output.weight")
            for b in ("attn_q", "attn_k", "attn_v", "attn_qkv", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                if p + b + ".bias" in w:
                    L.bias[b] = _as_f32(w[p + b + ".bias"])
            if cfg.num_experts:
                L.router = need(p + "ffn_gate_inp.weight")
                L.experts, L.expert_type = _expert_views(cfg, {s: need(p + f"ffn_{s}_exps.weight")
                                                               for s in ("gate", "up", "down")})
            else:
                L.gate, L.up, L.down = need(p + "ffn_gate.weight"), need(p + "ffn_up.weight"), need(p + "ffn_down.weight")
            self.layers.append(L)
        self.weights = w

    # -- sequences -------------------------------------------------------
    def new_sequence(self) -> int:
        free = set(range(self.max_num_seqs)) - set(self._slots.values())
        if not free:
            raise KVCacheError(f"all {self.max_num_seqs} sequence slots are in use")
        seq_id = self._next_seq_id
        self._next_seq_id += 1
        self._slots[seq_id] = min(free)
        self._length[seq_id] = 0
        return seq_id

    def end_sequence(self, seq_id: int) -> None:
        self._slots.pop(seq_id, None)
        self._length.pop(seq_id, None)

    def truncate_sequence(self, seq_id: int, new_length: int) -> None:
        if not 0 <= new_length <= self._length[seq_id]:
            raise KVCacheError(f"cannot truncate sequence {seq_id} of length {self._length[seq_id]} to {new_length}")
        self._length[seq_id] = int(new_length)

    # -- steps -----------------------------------------------------------
    def forward_step(self, seq_id: int, token_ids, start_position: int,
                     return_all_positions: bool = False) -> np.ndarray:
        ids = [int(t) for t in np.asarray(token_ids).reshape(-1)]
        if not ids:
            raise CPUError("forward_step needs at least one token")
        outs = []
        for j, tok in enumerate(ids):
            last = j == len(ids) - 1
            lg = self._step([seq_id], [tok], [start_position + j], logits=last or return_all_positions)
            if lg is not None:
                outs.append(lg)
        if return_all_positions:
            return torch.cat(outs, 0).cpu().numpy()
        return outs[-1][0].cpu().numpy()

    def forward_batch_decode(self, seq_ids: Sequence[int], token_ids: Sequence[int],
                             positions: Sequence[int]) -> np.ndarray:
        n = len(seq_ids)
        if not (len(token_ids) == len(positions) == n):
            raise CPUError("seq_ids, token_ids, and positions must be the same length.")
        outs = []
        for c in range(0, n, GEMV_MAX_M):
            outs.append(self._step(list(seq_ids[c:c + GEMV_MAX_M]), [int(t) for t in token_ids[c:c + GEMV_MAX_M]],
                                   [int(p) for p in positions[c:c + GEMV_MAX_M]], logits=True))
        return torch.cat(outs, 0).cpu().numpy()

    def generate_greedy(self, prompt_ids: Sequence[int], max_new_tokens: int) -> List[int]:
        seq_id = self.new_sequence()
        try:
            all_ids = list(prompt_ids)
            logits = self.forward_step(seq_id, np.array(all_ids, dtype=np.int64), start_position=0)
            for _ in range(max_new_tokens):
                nxt = int(np.argmax(logits))
                all_ids.append(nxt)
                logits = self.forward_step(seq_id, np.array([nxt]), start_position=len(all_ids) - 1)
            return all_ids
        finally:
            self.end_sequence(seq_id)

    def _step(self, seq_ids: List[int], tokens: List[int], positions: List[int], logits: bool):
        """One token for each of m <= 16 sequences; float32 logits [m, vocab] on the device (or None)."""
        cfg = self.config
        m = len(seq_ids)
        for s, p in zip(seq_ids, positions):
            if s not in self._slots:
                raise KVCacheError(f"unknown sequence {s}")
            if p != self._length[s]:
                raise KVCacheError(f"sequence {s} holds {self._length[s]} tokens; the next token's position must "
                                   f"be {self._length[s]}, got {p}")
            if p >= self.max_positions:
                raise KVCacheError(f"sequence {s} is full ({self.max_positions} positions)")
        for t in tokens:
            if not 0 <= t < self.embed.n:
                raise CPUError(f"token id {t} outside the vocabulary of {self.embed.n}")
        dev = self.device
        f32 = dict(dtype=torch.float32, device=dev)
        hd, hq, hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
        ids = torch.tensor(tokens, dtype=torch.int32, device=dev)
        # one 16-byte row per sequence: each sequence's position is its own aligned [1] view
        pos = torch.zeros((m, 4), dtype=torch.int32)
        pos[:, 0] = torch.tensor(positions, dtype=torch.int32)
        pos = pos.to(dev)
        h = torch.empty((m, cfg.hidden_size), **f32)
        get_rows(self.embed.data, self.embed.ggml_type, self.embed.shape, ids, out=h)
        xn = torch.empty_like(h)
        att = torch.empty((m, hq * hd), **f32)
        for li, L in enumerate(self.layers):
            rms_norm(h, L.attn_norm, cfg.rms_norm_eps, out=xn)
            q, k, v = self._qkv(L, xn)
            for i, s in enumerate(seq_ids):
                slot = self._slots[s]
                decode_attention(q[i:i + 1], k[i:i + 1], v[i:i + 1], self.k_cache[li][slot:slot + 1],
                                 self.v_cache[li][slot:slot + 1], pos[i, :1], hq, hkv, rope=self.rope,
                                 out=att[i:i + 1], workspace=self.attn_ws)
            self._linear(L.o, att, h, bias=L.bias.get("attn_output"), accumulate=True)
            rms_norm(h, L.ffn_norm, cfg.rms_norm_eps, out=xn)
            if L.experts is not None:
                self._moe(L, xn, h)
            else:
                self._mlp(L, xn, h)
        for s in seq_ids:
            self._length[s] += 1
        if not logits:
            return None
        rms_norm(h, self.output_norm, cfg.rms_norm_eps, out=xn)
        return self._linear(self.lm_head, xn, torch.empty((m, self.lm_head.n), **f32))

    # -- pieces ----------------------------------------------------------
    def _linear(self, w: DeviceWeight, x: torch.Tensor, out: torch.Tensor, bias=None, accumulate=False):
        """out (=|+=) x @ W.T (+ bias), x float32 [m, K]."""
        m = x.shape[0]
        if w.kind == "block":
            if accumulate and bias is None and m <= GEMV_MAX_M:
                gguf_gemv_residual(x, w.data, w.ggml_type, w.shape, out)
            elif accumulate:
                out.add_(gguf_linear(x, w.data, w.ggml_type, w.shape, bias=bias))
            else:
                gguf_linear(x, w.data, w.ggml_type, w.shape, bias=bias, out=out)
            return out
        if w.kind == "float":
            return dense_linear(x, w.data, w.ggml_type, w.shape, bias=bias, out=out, accumulate=accumulate)
        if w.kind == "flat":
            return dense_linear(x, w.dense, 0, w.shape, bias=bias, out=out, accumulate=accumulate)
        raise DracoFormatError(f"tensor '{w.name}' ({w.kind}) is not a 2-D weight")

    def _qkv(self, L: _Layer, xn: torch.Tensor):
        cfg = self.config
        m, hd = xn.shape[0], cfg.head_dim
        qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
        f32 = dict(dtype=torch.float32, device=self.device)
        if L.qkv is not None:
            qkv = self._linear(L.qkv, xn, torch.empty((m, qd + 2 * kvd), **f32), bias=L.bias.get("attn_qkv"))
            # one row per attention call: each row's slices are contiguous
            return qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:]
        q, k, v = torch.empty((m, qd), **f32), torch.empty((m, kvd), **f32), torch.empty((m, kvd), **f32)
        ws = (L.q, L.k, L.v)
        if (not L.bias and all(w.kind == "block" for w in ws) and len({w.ggml_type for w in ws}) == 1
                and m <= GEMV_MAX_M):
            gguf_gemv_multi(xn, [(w.data, w.n) for w in ws], L.q.ggml_type, cfg.hidden_size, [q, k, v])
        else:
            for w, o, b in ((L.q, q, "attn_q"), (L.k, k, "attn_k"), (L.v, v, "attn_v")):
                self._linear(w, xn, o, bias=L.bias.get(b))
        return q, k, v

    def _mlp(self, L: _Layer, xn: torch.Tensor, h: torch.Tensor) -> None:
        m = xn.shape[0]
        inter = L.gate.n
        s = torch.empty((m, inter), dtype=torch.float32, device=self.device)
        if (L.gate.kind == L.up.kind == "block" and L.gate.ggml_type == L.up.ggml_type and m <= GEMV_MAX_M
                and "ffn_gate" not in L.bias and "ffn_up" not in L.bias):
            gguf_gemv_swiglu(xn, L.gate.data, L.up.data, L.gate.ggml_type, L.gate.shape, out=s)
        else:
            g = self._linear(L.gate, xn, torch.empty_like(s), bias=L.bias.get("ffn_gate"))
            u = self._linear(L.up, xn, torch.empty_like(s), bias=L.bias.get("ffn_up"))
            swiglu(g, u, out=s)
        self._linear(L.down, s, h, bias=L.bias.get("ffn_down"), accumulate=True)

    def _moe(self, L: _Layer, xn: torch.Tensor, h: torch.Tensor) -> None:
        cfg = self.config
        m = xn.shape[0]
        logits = self._linear(L.router, xn, torch.empty((m, cfg.num_experts), dtype=torch.float32,
                                                         device=self.device))
        y = gguf_moe(xn, logits, L.experts["gate"], L.experts["up"], L.experts["down"], L.expert_type,
                     L.experts["inter"], top_k=cfg.num_experts_per_tok)
        h.add_(y)

    def close(self) -> None:
        if self._own_reader:
            self.reader.close()


def _as_f32(w: DeviceWeight) -> torch.Tensor:
    """A float tensor's values as contiguous float32 on the device (norm weights, biases)."""
    dt = {0: torch.float32, 1: torch.float16, 30: torch.bfloat16}[w.ggml_type]
    return w.data.view(dt).to(torch.float32).reshape(-1).contiguous()


def _expert_views(cfg: GPUExecutorConfig, stacks: Dict[str, DeviceWeight]):
    """Per-expert [rows, cols] byte views into the 3-D ``ffn_*_exps`` stacks
    (GGUF dims (cols, rows, n_experts): numpy shape (n_experts, rows, cols))."""
    g, u, d = stacks["gate"], stacks["up"], stacks["down"]
    types = {g.ggml_type, u.ggml_type, d.ggml_type}
    if len(types) != 1 or any(w.kind != "stack" or len(w.shape) != 3 for w in (g, u, d)):
        raise DracoFormatError("MoE expert stacks must be 3-D block tensors of one ggml type")
    ne, inter, hidden = g.shape
    if ne != cfg.num_experts or tuple(u.shape) != (ne, inter, hidden) or tuple(d.shape) != (ne, hidden, inter):
        raise DracoFormatError(f"expert stacks {g.shape} / {u.shape} / {d.shape} do not match {cfg.num_experts} "
                               f"experts of hidden {cfg.hidden_size}")
    eb = tensor_bytes(g.ggml_type, (inter, hidden))
    views = {"inter": inter}
    for key, w in (("gate", g), ("up", u), ("down", d)):
        parts = [w.data[e * eb:(e + 1) * eb] for e in range(ne)]
        if any(p.data_ptr() % 16 for p in parts):  # keep every expert 16-byte aligned for the kernels
            parts = [p.clone() for p in parts]
        views[key] = parts
    return views, next(iter(types))
