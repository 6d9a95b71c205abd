"""numpy restatement of the reference's decode-step glue (oracle only).

Follows the reference CPU runtime:

* ``rms_norm``          -> ``draco/runtime/cpu/ops.py:15-19``
  ``x32 / sqrt(mean(x32 * x32) + eps) * weight`` in float32.
* ``build_rope_cache``  -> ``draco/runtime/cpu/ops.py:73-79``
  ``inv_freq = 1 / theta ** (arange(0, D, 2) / D)``, ``freqs = pos x inv_freq``,
  cos / sin tables, float32.
* ``apply_rope``        -> ``draco/runtime/cpu/ops.py:82-92``
  half-split rotation: ``(x1 c - x2 s, x2 c + x1 s)`` with x1 / x2 the two
  halves of a head.
* ``decode attention``  -> ``draco/runtime/cpu/attention.py:35-81``
  (``prefill`` with one query, ``decode`` calls it with ``causal=False``): the
  new k / v are appended to the cache (stored in the cache dtype, float16 by
  default, ``draco/runtime/cpu/kv_cache.py:19-28``), cached keys / values are
  read back as float32 and repeated over the query-head groups (GQA),
  ``scores = q . k / sqrt(D)``, ``softmax`` (``ops.py:68-71``), ``probs @ v``.

``*_f64`` variants are fp64 closed forms used as the checker where the
float32 evaluation order of the GPU kernels differs from numpy's.
"""

from __future__ import annotations

from typing import Tuple

import numpy as np


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x32 = x.astype(np.float32)
    variance = np.mean(x32 * x32, axis=-1, keepdims=True)
    normed = x32 / np.sqrt(variance + eps)
    return (normed * weight).astype(x.dtype)


def rms_norm_f64(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x64 = np.asarray(x, dtype=np.float64)
    var = np.mean(x64 * x64, axis=-1, keepdims=True)
    return x64 / np.sqrt(var + eps) * np.asarray(weight, dtype=np.float64)


def rope_tables(head_dim: int, positions: np.ndarray, theta: float = 10000.0) -> Tuple[np.ndarray, np.ndarray]:
    """cos / sin [len(positions), head_dim // 2], float32 as the reference builds them."""
    inv_freq = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim))
    freqs = np.outer(np.asarray(positions, dtype=np.float32), inv_freq)
    return np.cos(freqs), np.sin(freqs)


def rope_tables_f64(head_dim: int, positions: np.ndarray, theta: float = 10000.0) -> Tuple[np.ndarray, np.ndarray]:
    inv_freq = 1.0 / (float(theta) ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    freqs = np.outer(np.asarray(positions, dtype=np.float64), inv_freq)
    return np.cos(freqs), np.sin(freqs)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [..., heads, D] for one position; cos / sin [D // 2] of that position."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1)


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    x = x - np.max(x, axis=axis, keepdims=True)
    e = np.exp(x)
    return e / np.sum(e, axis=axis, keepdims=True)


def decode_attention_f64(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, n_keys: int) -> np.ndarray:
    """One query token.  q [Hq, D] (RoPE applied); k_cache / v_cache [Hkv, >= n_keys, D]
    (the values the cache holds, i.e. float16-rounded); returns [Hq, D] in fp64."""
    hq, d = q.shape
    hkv = k_cache.shape[0]
    group = hq // hkv
    out = np.empty((hq, d), dtype=np.float64)
    for h in range(hq):
        kk = np.asarray(k_cache[h // group, :n_keys], dtype=np.float64)
        vv = np.asarray(v_cache[h // group, :n_keys], dtype=np.float64)
        s = kk @ np.asarray(q[h], dtype=np.float64) / np.sqrt(d)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vv
    return out


def decode_step_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                          pos: int, theta: float, rope: bool = True) -> np.ndarray:
    """The reference decode attention for one sequence, in place on the cache.

    q [Hq, D], k / v [Hkv, D] float32 projections of the new token (before
    RoPE); k_cache / v_cache float16 [Hkv, max_pos, D] holding positions
    0 .. pos - 1.  Rotates q and k with the position-``pos`` tables, stores k
    and v at ``pos`` (float16), and returns the attention output [Hq, D] in
    fp64 over the ``pos + 1`` cached keys."""
    if rope:
        cos, sin = rope_tables_f64(q.shape[-1], np.array([pos]), theta)
        q = apply_rope(q.astype(np.float64), cos[0], sin[0])
        k = apply_rope(k.astype(np.float64), cos[0], sin[0])
    k_cache[:, pos] = k.astype(np.float16)
    v_cache[:, pos] = v.astype(np.float16)
    return decode_attention_f64(q, k_cache, v_cache, pos + 1)
