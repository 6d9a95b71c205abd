"""Seeded GGUF test inputs shared by the GPU parity tests.

Weights are N(0, 0.02) float32 with a seeded 1 % of rows scaled x4, quantized
on the CPU by the package's quantizers (Q8_0 / Q4_0 bytes equal the
reference's test encoders; Q4_K / Q6_K are this package's encoders); the
expected float32 weight is the oracle's dequantization of those same bytes.
"""

from __future__ import annotations

import functools

import numpy as np
import torch

from dracort_amd.quantization import quantize
from oracle import gguf_ref, matmul_ref

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K, Q8_K = 3, 6, 7, 10, 11, 13, 15
GGML_ORDER = 0x100
TYPES = [Q8_0, Q4_0, Q4_K, Q6_K]
MORE_TYPES = [Q4_1, Q5_0, Q5_1, Q8_K, Q2_K, Q3_K, Q5_K]
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1",
         Q2_K: "Q2_K", Q3_K: "Q3_K", Q5_K: "Q5_K", Q8_K: "Q8_K"}


def qk_of(qtype: int) -> int:
    return gguf_ref.BLOCK_LAYOUT[qtype & ~GGML_ORDER][0]


def type_name(qtype: int) -> str:
    return NAMES[qtype & ~GGML_ORDER] + ("/ggml-order" if qtype & GGML_ORDER else "")
TOL = 1e-3  # max elementwise relative error vs the fp64 closed form (floor 1e-3 * max|ref|)


def synth_weight(n: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    rows = rng.choice(n, size=max(1, n // 100), replace=False)
    w[rows] *= 4.0
    return w


@functools.lru_cache(maxsize=16)
def quantized(qtype: int, n: int, k: int, seed: int = 0):
    """(packed bytes uint8 [nbytes], oracle float32 dequant [n, k])"""
    w = synth_weight(n, k, seed)
    blocks = quantize(torch.from_numpy(w), qtype).numpy()
    base = qtype & ~0x100
    return blocks, gguf_ref.dequantize_matrix(base, blocks, (n, k), ggml_order=bool(qtype & 0x100))


def activations(m: int, k: int, seed: int, dtype: torch.dtype) -> torch.Tensor:
    rng = np.random.default_rng(seed + 1000)
    x = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32))
    return x.to(dtype)


def check_close(y: np.ndarray, ref: np.ndarray, what: str, tol: float = TOL):
    elem, norm = matmul_ref.rel_err(y, ref)
    assert elem <= tol, f"{what}: max rel err {elem:.3e} (normwise {norm:.3e}) > {tol}"
    return elem, norm
