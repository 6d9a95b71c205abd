"""GGUF block quantizers (torch; run on the GPU or the CPU).

* ``quantize_q8_0`` / ``quantize_q4_0`` produce the same bytes as the
  reference's only GGUF encoders, its test helpers ``_enc_q8_0`` /
  ``_enc_q4_0`` (``tests/format/test_gguf.py:145-169``): block scale
  ``max(amax, 1e-12) / 127`` (``/ 8`` for Q4_0) in float32, codes rounded
  half-to-even with that float32 scale, the float16 rounding of the scale
  stored; Q4_0 codes ``clip(rint(x/d) + 8, 0, 15)``, low nibbles = elements
  0..15, high nibbles = 16..31.
* ``quantize_q4_k`` / ``quantize_q6_k`` are this package's own: the reference
  has no K-quant encoder.  They write the reference's block layouts
  (``draco/format/gguf.py:84-86``): Q4_K = f16 d, f16 dmin, 12 packed 6-bit
  scale/min bytes, 128 nibble bytes; Q6_K = f16 d, ql[128], qh[64], int8
  scales[16] (``d_last=True`` writes the upstream order with d last).
  Q4_K: per 32-weight sub-block, min' = -min(0, min x) and
  scale = (max x + min') / 15; d = max scale / 63, dmin = max min' / 63 (as
  float16); sub-block scales and mins rounded to 6 bits against them; codes
  ``clamp(rint((x + dmin*m) / (d*sc)), 0, 15)``.
  Q6_K: per 16-weight sub-block s = amax / 31; d = max |s| / 127 (float16);
  int8 scales ``rint(s / d)``; codes ``clamp(rint(x / (d*sc)), -32, 31) + 32``.

Weights are [N, K] with K a multiple of the block size; the result is a flat
uint8 tensor of N * K/QK blocks on the input's device.
"""

from __future__ import annotations

import torch

from dracort_amd.format.gguf import (
    GGML_TYPE_Q4_0,
    GGML_TYPE_Q4_K,
    GGML_TYPE_Q6_K,
    GGML_TYPE_Q8_0,
    Q6K_D_LAST,
    base_type,
    row_bytes,
)


def _f16_bytes(v: torch.Tensor) -> torch.Tensor:
    """float32 [B] -> uint8 [B, 2] little-endian float16 bits."""
    bits = v.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    return torch.stack([bits & 0xFF, bits >> 8], dim=-1).to(torch.uint8)


def _blocks(w: torch.Tensor, qk: int) -> torch.Tensor:
    if w.dim() != 2 or w.shape[1] % qk != 0:
        raise ValueError(f"weight must be [N, K] with K a multiple of {qk}, got {tuple(w.shape)}")
    return w.to(torch.float32).contiguous().reshape(-1, qk)


def quantize_q8_0(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 32)
    scale = torch.clamp(a.abs().amax(dim=1), min=1e-12) / 127.0
    codes = torch.clamp(torch.round(a / scale[:, None]), -127, 127).to(torch.int8)
    out = torch.empty((a.shape[0], 34), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(scale)
    out[:, 2:34] = codes.view(torch.uint8)
    return out.reshape(-1)


def quantize_q4_0(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 32)
    scale = torch.clamp(a.abs().amax(dim=1), min=1e-12) / 8.0
    codes = torch.clamp(torch.round(a / scale[:, None]) + 8, 0, 15).to(torch.uint8)
    out = torch.empty((a.shape[0], 18), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(scale)
    out[:, 2:18] = codes[:, 0:16] | (codes[:, 16:32] << 4)
    return out.reshape(-1)


def quantize_q4_k(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 256).reshape(-1, 8, 32)
    nb = a.shape[0]
    neg_min = torch.clamp(a.amin(dim=2), max=0.0).neg()           # >= 0
    scale = (a.amax(dim=2) + neg_min) / 15.0                       # >= 0
    d = (scale.amax(dim=1) / 63.0).to(torch.float16).to(torch.float32)
    dmin = (neg_min.amax(dim=1) / 63.0).to(torch.float16).to(torch.float32)
    sc = torch.where(d[:, None] > 0, torch.round(scale / d[:, None]), torch.zeros_like(scale)).clamp(0, 63)
    mn = torch.where(dmin[:, None] > 0, torch.round(neg_min / dmin[:, None]), torch.zeros_like(neg_min)).clamp(0, 63)
    d1 = d[:, None] * sc
    m1 = dmin[:, None] * mn
    safe = torch.where(d1 > 0, d1, torch.ones_like(d1))
    q = torch.round((a + m1[:, :, None]) / safe[:, :, None]).clamp(0, 15)
    q = torch.where(d1[:, :, None] > 0, q, torch.zeros_like(q)).to(torch.uint8)
    sc = sc.to(torch.uint8)
    mn = mn.to(torch.uint8)
    packed = torch.empty((nb, 12), dtype=torch.uint8, device=a.device)
    packed[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    packed[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    packed[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    qp = q.reshape(nb, 4, 2, 32)
    qs = qp[:, :, 0, :] | (qp[:, :, 1, :] << 4)                     # [nb, 4, 32]
    out = torch.empty((nb, 144), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(d)
    out[:, 2:4] = _f16_bytes(dmin)
    out[:, 4:16] = packed
    out[:, 16:144] = qs.reshape(nb, 128)
    return out.reshape(-1)


def quantize_q6_k(w: torch.Tensor, d_last: bool = False) -> torch.Tensor:
    a = _blocks(w, 256)
    nb = a.shape[0]
    sub = a.reshape(nb, 16, 16)
    s = sub.abs().amax(dim=2) / 31.0                               # [nb, 16] >= 0
    d = (s.amax(dim=1) / 127.0).to(torch.float16).to(torch.float32)
    sc = torch.where(d[:, None] > 0, torch.round(s / d[:, None]), torch.zeros_like(s)).clamp(-128, 127)
    dl = d[:, None] * sc
    safe = torch.where(dl != 0, dl, torch.ones_like(dl))
    q = torch.round(sub / safe[:, :, None]).clamp(-32, 31)
    q = torch.where(dl[:, :, None] != 0, q, torch.zeros_like(q))
    q = (q + 32).to(torch.int32).reshape(nb, 2, 4, 32)              # [nb, half, t, l]
    lo = q & 15
    hi = q >> 4
    ql = torch.empty((nb, 2, 64), dtype=torch.int32, device=a.device)
    ql[:, :, 0:32] = lo[:, :, 0] | (lo[:, :, 2] << 4)
    ql[:, :, 32:64] = lo[:, :, 1] | (lo[:, :, 3] << 4)
    qh = hi[:, :, 0] | (hi[:, :, 1] << 2) | (hi[:, :, 2] << 4) | (hi[:, :, 3] << 6)   # [nb, 2, 32]
    sc8 = sc.to(torch.int8).view(torch.uint8)
    out = torch.empty((nb, 210), dtype=torch.uint8, device=a.device)
    if d_last:
        out[:, 0:128] = ql.reshape(nb, 128).to(torch.uint8)
        out[:, 128:192] = qh.reshape(nb, 64).to(torch.uint8)
        out[:, 192:208] = sc8
        out[:, 208:210] = _f16_bytes(d)
    else:
        out[:, 0:2] = _f16_bytes(d)
        out[:, 2:130] = ql.reshape(nb, 128).to(torch.uint8)
        out[:, 130:194] = qh.reshape(nb, 64).to(torch.uint8)
        out[:, 194:210] = sc8
    return out.reshape(-1)


def quantize(w: torch.Tensor, ggml_type: int) -> torch.Tensor:
    """Quantize an [N, K] float weight to GGUF blocks of ``ggml_type``."""
    base = base_type(ggml_type)
    row_bytes(ggml_type, int(w.shape[-1]))  # validates type and K
    if base == GGML_TYPE_Q8_0:
        return quantize_q8_0(w)
    if base == GGML_TYPE_Q4_0:
        return quantize_q4_0(w)
    if base == GGML_TYPE_Q4_K:
        return quantize_q4_k(w)
    return quantize_q6_k(w, d_last=bool(int(ggml_type) & Q6K_D_LAST))
