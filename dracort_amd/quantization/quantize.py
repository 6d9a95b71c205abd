"""GGUF block quantizers (torch; run on the GPU or the CPU).

* ``quantize_q8_0`` / ``quantize_q4_0`` / ``quantize_q4_1`` /
  ``quantize_q5_0`` / ``quantize_q5_1`` produce the same bytes as the
  reference's only GGUF encoders, its test helpers ``_enc_q8_0`` ...
  ``_enc_q5_1`` (``tests/format/test_gguf.py:145-229``): block scale
  ``max(amax, 1e-12) / 127`` (``/ 8`` Q4_0, ``/ 16`` Q5_0) or
  ``(max - min) / 15`` (``/ 31`` Q5_1; 1 when the span is <= 1e-12, offset
  ``min``) in float32, codes rounded half-to-even with that float32 scale, the
  float16 rounding of the scale (and offset) stored; low nibbles = elements
  0..15, high nibbles = 16..31; Q5 fifth bits at bit e of the qh word.
* The K-quants and Q8_K are this package's own: the reference has no
  K-quant encoder.  They write the reference's block layouts
  (``draco/format/gguf.py:75-87``; ``GGML_ORDER`` writes Q2_K / Q3_K / Q6_K
  in upstream ggml field order instead):
  Q4_K / Q5_K: per 32-weight sub-block, min' = -min(0, min x) and
  scale = (max x + min') / 15 (/ 31); d = max scale / 63, dmin = max min' / 63
  (as float16); 6-bit sub-block scales and mins against them; codes
  ``clamp(rint((x + dmin*m) / (d*sc)), 0, 15 | 31)``.
  Q2_K: the same per 16-weight run with 2-bit codes and 4-bit scales / mins
  (d = max scale / 15, dmin = max min' / 15).
  Q3_K: per 16-weight run s = amax / 4; d = max s / 31; scales
  ``rint(s / d) + 32`` (6 bits); codes ``clamp(rint(x / (d*(sc-32))), -4, 3) + 4``.
  Q6_K: per 16-weight run s = amax / 31; d = max |s| / 127 (float16);
  int8 scales ``rint(s / d)``; codes ``clamp(rint(x / (d*sc)), -32, 31) + 32``.
  Q8_K: per 256-weight block d = max(amax, 1e-12) / 127, codes
  ``clamp(rint(x / d), -127, 127)`` with the float32 d, float16 d stored.

Weights are [N, K] with K a multiple of the block size; the result is a flat
uint8 tensor of N * K/QK blocks on the input's device.
"""

from __future__ import annotations

import torch

from dracort_amd.format.gguf import (
    GGML_ORDER,
    GGML_TYPE_Q2_K,
    GGML_TYPE_Q3_K,
    GGML_TYPE_Q4_0,
    GGML_TYPE_Q4_1,
    GGML_TYPE_Q4_K,
    GGML_TYPE_Q5_0,
    GGML_TYPE_Q5_1,
    GGML_TYPE_Q5_K,
    GGML_TYPE_Q6_K,
    GGML_TYPE_Q8_0,
    GGML_TYPE_Q8_K,
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


def _nibbles(codes: torch.Tensor) -> torch.Tensor:
    """[B, 32] codes -> [B, 16] bytes: low nibbles elements 0..15, high 16..31."""
    return ((codes[:, 0:16] & 15) | ((codes[:, 16:32] & 15) << 4)).to(torch.uint8)


def _fifth_bits(codes: torch.Tensor) -> torch.Tensor:
    """[B, 32] codes -> [B, 4] bytes of the qh word (bit e = bit 4 of code e)."""
    bits = ((codes >> 4) & 1).to(torch.int64).reshape(-1, 4, 8)
    weights = (1 << torch.arange(8, device=codes.device, dtype=torch.int64))
    return (bits * weights).sum(dim=2).to(torch.uint8)


def _affine(a: torch.Tensor, top: int):
    lo = a.amin(dim=1)
    span = a.amax(dim=1) - lo
    d = torch.where(span > 1e-12, span / float(top), torch.ones_like(span))
    codes = torch.clamp(torch.round((a - lo[:, None]) / d[:, None]), 0, top).to(torch.int32)
    return d, lo, codes


def quantize_q4_1(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 32)
    d, lo, codes = _affine(a, 15)
    out = torch.empty((a.shape[0], 20), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(d)
    out[:, 2:4] = _f16_bytes(lo)
    out[:, 4:20] = _nibbles(codes)
    return out.reshape(-1)


def quantize_q5_0(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 32)
    d = torch.clamp(a.abs().amax(dim=1), min=1e-12) / 16.0
    codes = torch.clamp(torch.round(a / d[:, None]) + 16, 0, 31).to(torch.int32)
    out = torch.empty((a.shape[0], 22), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(d)
    out[:, 2:6] = _fifth_bits(codes)
    out[:, 6:22] = _nibbles(codes)
    return out.reshape(-1)


def quantize_q5_1(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 32)
    d, lo, codes = _affine(a, 31)
    out = torch.empty((a.shape[0], 24), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(d)
    out[:, 2:4] = _f16_bytes(lo)
    out[:, 4:8] = _fifth_bits(codes)
    out[:, 8:24] = _nibbles(codes)
    return out.reshape(-1)


def quantize_q8_k(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 256)
    d = torch.clamp(a.abs().amax(dim=1), min=1e-12) / 127.0
    codes = torch.clamp(torch.round(a / d[:, None]), -127, 127).to(torch.int8)
    out = torch.empty((a.shape[0], 258), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(d)
    out[:, 2:258] = codes.view(torch.uint8)
    return out.reshape(-1)


def _scale_min_runs(sub: torch.Tensor, levels: int, scale_max: int):
    """Asymmetric runs [B, R, L]: (d, dmin) float16-exact, per-run integer
    scale / min in 0..scale_max, codes in 0..levels."""
    neg_min = torch.clamp(sub.amin(dim=2), max=0.0).neg()
    scale = (sub.amax(dim=2) + neg_min) / float(levels)
    d = (scale.amax(dim=1) / float(scale_max)).to(torch.float16).to(torch.float32)
    dmin = (neg_min.amax(dim=1) / float(scale_max)).to(torch.float16).to(torch.float32)
    sc = torch.where(d[:, None] > 0, torch.round(scale / d[:, None]), torch.zeros_like(scale)).clamp(0, scale_max)
    mn = torch.where(dmin[:, None] > 0, torch.round(neg_min / dmin[:, None]),
                     torch.zeros_like(neg_min)).clamp(0, scale_max)
    d1 = d[:, None] * sc
    m1 = dmin[:, None] * mn
    safe = torch.where(d1 > 0, d1, torch.ones_like(d1))
    q = torch.round((sub + m1[:, :, None]) / safe[:, :, None]).clamp(0, levels)
    q = torch.where(d1[:, :, None] > 0, q, torch.zeros_like(q)).to(torch.int32)
    return d, dmin, sc.to(torch.int32), mn.to(torch.int32), q


def _pack_k4_scales(sc: torch.Tensor, mn: torch.Tensor) -> torch.Tensor:
    """8 six-bit (scale, min) pairs -> the 12 packed bytes of Q4_K / Q5_K."""
    packed = torch.empty((sc.shape[0], 12), dtype=torch.int32, device=sc.device)
    packed[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    packed[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    packed[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    return packed.to(torch.uint8)


def quantize_q5_k(w: torch.Tensor) -> torch.Tensor:
    a = _blocks(w, 256).reshape(-1, 8, 32)
    nb = a.shape[0]
    d, dmin, sc, mn, q = _scale_min_runs(a, 31, 63)
    qp = q.reshape(nb, 4, 2, 32)
    qs = (qp[:, :, 0, :] & 15) | ((qp[:, :, 1, :] & 15) << 4)                     # [nb, 4, 32]
    fifth = (q >> 4) & 1                                                            # [nb, 8 sub-blocks, 32]
    qh = (fifth << torch.arange(8, device=a.device, dtype=torch.int32)[None, :, None]).sum(dim=1)
    out = torch.empty((nb, 176), dtype=torch.uint8, device=a.device)
    out[:, 0:2] = _f16_bytes(d)
    out[:, 2:4] = _f16_bytes(dmin)
    out[:, 4:16] = _pack_k4_scales(sc, mn)
    out[:, 16:48] = qh.to(torch.uint8)
    out[:, 48:176] = qs.reshape(nb, 128).to(torch.uint8)
    return out.reshape(-1)


def _runs_to_k6_bytes(q: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes [nb, 256] in element order -> [nb, 64] bytes: the low 2 bits of
    element (half, j, sub, l) at bits 2j of byte 32*half + 16*sub + l."""
    nb = q.shape[0]
    c = (q & 3).reshape(nb, 2, 4, 2, 16)                                            # half, j, sub, l
    shift = (2 * torch.arange(4, device=q.device, dtype=torch.int32)).reshape(1, 1, 4, 1, 1)
    return (c << shift).sum(dim=2).reshape(nb, 64).to(torch.uint8)


def quantize_q2_k(w: torch.Tensor, ggml_order: bool = False) -> torch.Tensor:
    a = _blocks(w, 256)
    nb = a.shape[0]
    d, dmin, sc, mn, q = _scale_min_runs(a.reshape(nb, 16, 16), 3, 15)
    qs = _runs_to_k6_bytes(q.reshape(nb, 256), 2)
    scb = (sc | (mn << 4)).to(torch.uint8)                                          # run r = element // 16
    out = torch.empty((nb, 84), dtype=torch.uint8, device=a.device)
    if ggml_order:
        out[:, 0:16], out[:, 16:80] = scb, qs
        out[:, 80:82], out[:, 82:84] = _f16_bytes(d), _f16_bytes(dmin)
    else:
        out[:, 0:2], out[:, 2:4] = _f16_bytes(d), _f16_bytes(dmin)
        out[:, 4:68], out[:, 68:84] = qs, scb
    return out.reshape(-1)


def quantize_q3_k(w: torch.Tensor, ggml_order: bool = False) -> torch.Tensor:
    a = _blocks(w, 256)
    nb = a.shape[0]
    sub = a.reshape(nb, 16, 16)
    s = sub.abs().amax(dim=2) / 4.0                                                 # [nb, 16] >= 0
    d = (s.amax(dim=1) / 31.0).to(torch.float16).to(torch.float32)
    sc = torch.where(d[:, None] > 0, torch.round(s / d[:, None]), torch.zeros_like(s)).clamp(0, 31)
    dl = d[:, None] * sc
    safe = torch.where(dl > 0, dl, torch.ones_like(dl))
    q = torch.round(sub / safe[:, :, None]).clamp(-4, 3)
    q = (torch.where(dl[:, :, None] > 0, q, torch.zeros_like(q)) + 4).to(torch.int32).reshape(nb, 256)
    qs = _runs_to_k6_bytes(q, 2)
    high = ((q >> 2) & 1).reshape(nb, 2, 4, 2, 16)                                  # half, j, sub, l
    bit = (4 * torch.arange(2, device=a.device, dtype=torch.int32)[:, None]
           + torch.arange(4, device=a.device, dtype=torch.int32)[None, :]).reshape(1, 2, 4, 1, 1)
    hm = (high << bit).sum(dim=(1, 2)).reshape(nb, 32).to(torch.uint8)              # byte 16*sub + l
    s6 = sc.to(torch.int32) + 32                                                    # run i = element // 16
    s12 = torch.zeros((nb, 12), dtype=torch.int32, device=a.device)
    for i in range(16):
        s12[:, i % 8] |= (s6[:, i] & 15) << (4 * (i // 8))
        s12[:, 8 + i % 4] |= (s6[:, i] >> 4) << (2 * (i // 4))
    s12 = s12.to(torch.uint8)
    out = torch.empty((nb, 110), dtype=torch.uint8, device=a.device)
    if ggml_order:
        out[:, 0:32], out[:, 32:96], out[:, 96:108], out[:, 108:110] = hm, qs, s12, _f16_bytes(d)
    else:
        out[:, 0:2], out[:, 2:14], out[:, 14:78], out[:, 78:110] = _f16_bytes(d), s12, qs, hm
    return out.reshape(-1)


def quantize(w: torch.Tensor, ggml_type: int) -> torch.Tensor:
    """Quantize an [N, K] float weight to GGUF blocks of ``ggml_type``."""
    base = base_type(ggml_type)
    row_bytes(ggml_type, int(w.shape[-1]))  # validates type, layout flag and K
    upstream = bool(int(ggml_type) & GGML_ORDER)
    simple = {GGML_TYPE_Q8_0: quantize_q8_0, GGML_TYPE_Q4_0: quantize_q4_0, GGML_TYPE_Q4_1: quantize_q4_1,
              GGML_TYPE_Q5_0: quantize_q5_0, GGML_TYPE_Q5_1: quantize_q5_1, GGML_TYPE_Q8_K: quantize_q8_k,
              GGML_TYPE_Q4_K: quantize_q4_k, GGML_TYPE_Q5_K: quantize_q5_k}
    if base in simple:
        return simple[base](w)
    if base == GGML_TYPE_Q2_K:
        return quantize_q2_k(w, ggml_order=upstream)
    if base == GGML_TYPE_Q3_K:
        return quantize_q3_k(w, ggml_order=upstream)
    return quantize_q6_k(w, d_last=upstream)
