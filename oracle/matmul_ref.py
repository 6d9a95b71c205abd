"""Closed-form references for the matmul, the MoE FFN and the acceptance metric
(oracle only).

* ``linear_ref``     ``x @ W.T`` in float64 from the bit-exact float32 dequant;
                     the reference computes it as
                     ``activation.astype(f32) @ weight.astype(f32).T``
                     (``draco/runtime/cpu/kernels/generic.py:32-33``) called from
                     ``_linear`` (``draco/runtime/cpu/executor.py:47-79``).
* ``cpu_linear_f32`` exactly the reference's float32 numpy expression; this is
                     the timed CPU baseline, not a checker.
* ``cpu_moe_f32``    the reference's MoE in float32 (top-k of the logits,
                     softmax, per-expert ``F.linear`` SwiGLU FFN on the tokens
                     routed to it, weighted sum) with numpy/OpenBLAS: the timed
                     CPU baseline of the MoE configuration, not a checker.
* ``moe_ref``        top-k router (``draco/models/moe/router.py:81-120``: topk of
                     the logits, softmax over the k selected logits, renormalise)
                     and the expert loop (``draco/models/moe/expert.py:77-116``:
                     experts in ascending order, ``down(silu(gate x) * up x)``,
                     weighted by the routing weight of the slot, summed into the
                     token's output), all in float64.
* ``rel_err``        max_i |y_i - r_i| / max(|r_i|, 1e-3 * max_j |r_j|): the
                     elementwise relative error with a floor for outputs near
                     zero, plus the normwise ||y - r|| / ||r||.
"""

from __future__ import annotations

from typing import Sequence, Tuple

import numpy as np


def linear_ref(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x64 = np.asarray(x, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float64)
    return x64 @ w64.T


def cpu_linear_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    return x.astype(np.float32, copy=False) @ w.astype(np.float32, copy=False).T


def rel_err(y: np.ndarray, ref: np.ndarray) -> Tuple[float, float]:
    y64 = np.asarray(y, dtype=np.float64)
    r64 = np.asarray(ref, dtype=np.float64)
    if r64.size == 0:
        return 0.0, 0.0
    scale = np.max(np.abs(r64))
    if scale == 0.0:
        e = float(np.max(np.abs(y64)))
        return e, e
    denom = np.maximum(np.abs(r64), 1e-3 * scale)
    elem = float(np.max(np.abs(y64 - r64) / denom))
    norm = float(np.linalg.norm(y64 - r64) / max(np.linalg.norm(r64), 1e-300))
    return elem, norm


def silu64(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def route_ref(logits: np.ndarray, top_k: int) -> Tuple[np.ndarray, np.ndarray]:
    """(expert index [T, k], routing weight [T, k]) in float64.

    Selection is by descending logit; equal logits go to the lower expert
    index (the reference's torch.topk leaves ties unspecified).
    """
    lg = np.asarray(logits, dtype=np.float64)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :top_k]
    top = np.take_along_axis(lg, order, axis=1)
    e = np.exp(top - top.max(axis=1, keepdims=True))
    w = e / e.sum(axis=1, keepdims=True)
    w = w / w.sum(axis=1, keepdims=True)
    return order, w


def moe_ref(
    x: np.ndarray,
    logits: np.ndarray,
    experts: Sequence[Tuple[np.ndarray, np.ndarray, np.ndarray]],
    top_k: int,
) -> np.ndarray:
    """experts[e] = (W_gate [I, H], W_up [I, H], W_down [H, I]) as float arrays."""
    x64 = np.asarray(x, dtype=np.float64)
    idx, w = route_ref(logits, top_k)
    out = np.zeros_like(x64)
    for e, (wg, wu, wd) in enumerate(experts):
        hit = np.nonzero((idx == e).any(axis=1))[0]
        if hit.size == 0:
            continue
        xe = x64[hit]
        h = silu64(xe @ np.asarray(wg, np.float64).T) * (xe @ np.asarray(wu, np.float64).T)
        ye = h @ np.asarray(wd, np.float64).T
        we = (w[hit] * (idx[hit] == e)).sum(axis=1, keepdims=True)
        out[hit] += ye * we
    return out


def cpu_moe_f32(x: np.ndarray, logits: np.ndarray, experts, top_k: int) -> np.ndarray:
    """float32 MoE FFN as the reference's modules compute it on the CPU (timed baseline)."""
    x32 = np.asarray(x, dtype=np.float32)
    idx, w = route_ref(logits, top_k)
    out = np.zeros_like(x32)
    for e, (wg, wu, wd) in enumerate(experts):
        hit = np.nonzero((idx == e).any(axis=1))[0]
        if hit.size == 0:
            continue
        xe = x32[hit]
        g = xe @ wg.T
        h = g / (1.0 + np.exp(-g)) * (xe @ wu.T)
        we = (w[hit] * (idx[hit] == e)).sum(axis=1, keepdims=True).astype(np.float32)
        out[hit] += (h @ wd.T) * we
    return out
