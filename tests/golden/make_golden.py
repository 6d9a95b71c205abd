"""Write the golden GGUF dequant / encoder vectors from the reference itself.

Run once, in the build container only (the reference tree is not present where
the tests run):

    python tests/golden/make_golden.py /root/reference

It imports ``draco.format.gguf`` behind a package stub (the same isolation the
reference's own ``tests/conftest.py:16-29`` uses, so ``draco/__init__.py`` and
its torch imports are not executed), and the reference test module for its
``_enc_q8_0`` / ``_enc_q4_0`` encoders (``tests/format/test_gguf.py:145-169``).
Only inputs and outputs are written (``gguf_dequant_golden.npz``,
``gguf_encoder_golden.npz``); no reference code is stored.

Inputs are seeded random blocks with finite float16 scales (normal, subnormal,
negative, zero, max-magnitude) and random code/scale bytes, so every nibble,
6-bit scale path and sign is exercised.  NaN/Inf scales are excluded: their
payload propagation is not part of the parity contract.
"""

from __future__ import annotations

import importlib.util
import os
import sys
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

TYPES = {"Q4_0": (2, 32, 18), "Q8_0": (8, 32, 34), "Q4_K": (12, 256, 144), "Q6_K": (14, 256, 210)}
# byte offsets of float16 fields inside a block, in the reference's layout
F16_FIELDS = {"Q4_0": [0], "Q8_0": [0], "Q4_K": [0, 2], "Q6_K": [0]}
N_BLOCKS = {"Q4_0": 192, "Q8_0": 192, "Q4_K": 48, "Q6_K": 48}


def _import_reference(ref_root: str):
    draco_dir = os.path.join(ref_root, "draco")
    for name, sub in (("draco", ""), ("draco.format", "format")):
        if name not in sys.modules:
            mod = types.ModuleType(name)
            mod.__path__ = [os.path.join(draco_dir, sub)]
            sys.modules[name] = mod
    from draco.format import gguf  # noqa: E402

    spec = importlib.util.spec_from_file_location(
        "_ref_test_gguf", os.path.join(ref_root, "tests", "format", "test_gguf.py")
    )
    tmod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(tmod)
    return gguf, tmod


def _f16_pool(rng: np.random.Generator, n: int) -> np.ndarray:
    """Finite float16 bit patterns covering every class the parity contract includes."""
    normal = (rng.normal(size=n) * 0.02).astype(np.float16)
    wide = (rng.normal(size=n) * 40.0).astype(np.float16)
    sub = rng.integers(1, 0x400, size=n, dtype=np.uint16) | (rng.integers(0, 2, size=n, dtype=np.uint16) << 15)
    special = np.array([0x0000, 0x8000, 0x7BFF, 0xFBFF, 0x0400, 0x3C00, 0xBC00, 0x0001], dtype=np.uint16)
    kind = rng.integers(0, 4, size=n)
    out = normal.view(np.uint16).copy()
    out[kind == 1] = wide.view(np.uint16)[kind == 1]
    out[kind == 2] = sub[kind == 2]
    pick = rng.integers(0, special.size, size=n)
    out[kind == 3] = special[pick][kind == 3]
    return out


def make_dequant(gguf) -> dict:
    rng = np.random.default_rng(20261201)
    out = {}
    for name, (gtype, qk, nbytes) in TYPES.items():
        nb = N_BLOCKS[name]
        blocks = rng.integers(0, 256, size=(nb, nbytes), dtype=np.uint8)
        for off in F16_FIELDS[name]:
            bits = _f16_pool(rng, nb)
            blocks[:, off] = (bits & 0xFF).astype(np.uint8)
            blocks[:, off + 1] = (bits >> 8).astype(np.uint8)
        payload = blocks.tobytes()
        expect = gguf._dequantize(gtype, payload, nb * qk)
        assert expect.dtype == np.float32 and np.all(np.isfinite(expect))
        out[f"{name}_blocks"] = blocks
        out[f"{name}_expect_bits"] = expect.view(np.uint32)
    return out


def make_encoders(tmod) -> dict:
    out = {}
    x_small = (np.random.default_rng(3).normal(size=64) * 2.0).astype(np.float32)
    x_wide = (np.random.default_rng(5).normal(size=4096) * 0.02).astype(np.float32)
    x_wide[::97] *= 4.0
    x_zero = np.zeros(64, dtype=np.float32)
    for tag, x in (("small", x_small), ("wide", x_wide), ("zero", x_zero)):
        out[f"x_{tag}"] = x
        out[f"q8_0_{tag}"] = np.frombuffer(tmod._enc_q8_0(x), dtype=np.uint8)
        out[f"q4_0_{tag}"] = np.frombuffer(tmod._enc_q4_0(x), dtype=np.uint8)
    return out


def main(ref_root: str) -> None:
    gguf, tmod = _import_reference(ref_root)
    np.savez_compressed(os.path.join(HERE, "gguf_dequant_golden.npz"), **make_dequant(gguf))
    np.savez_compressed(os.path.join(HERE, "gguf_encoder_golden.npz"), **make_encoders(tmod))
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
