"""GGUF file -> HBM upload in the native packed layout.

The reference keeps a GGUF tensor on the host and dequantizes it to float32
on first use (``GGUFReader.get_tensor``, ``draco/format/gguf.py:820-834``),
and its checkpoint loaders hand back host tensors
(``CheckpointLoader.register_loader``, ``draco/weights/loader.py:397-402``).
Here the packed blocks go to the device unchanged: the file's mapping is read
in chunks into two pinned host buffers that alternate, each chunk copied to
the device asynchronously on a dedicated stream while the next is being
filled, so disk / page-cache reads overlap the host-to-device copies.

Quantized 2-D tensors of a block type the kernels run, with whole blocks
per row, come back as :class:`GGUFQuantizedWeight`; float tensors (norms,
embeddings) as device tensors of their dtype and shape; everything else
(3-D expert stacks, tensors whose blocks run across rows) as raw uint8
bytes.
"""

from __future__ import annotations

from typing import Dict, Iterable, Optional, Union

import numpy as np
import torch

from dracort_amd.format.gguf import BLOCK_LAYOUTS, base_type
from dracort_amd.format.gguf_file import FLOAT_TYPES, GGUFFile
from dracort_amd.quantization.gguf import GGUFQuantizedWeight

_TORCH_FLOAT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}

Uploaded = Union[GGUFQuantizedWeight, torch.Tensor]


def upload_gguf(
    gguf: GGUFFile,
    names: Optional[Iterable[str]] = None,
    device: Union[str, torch.device] = "cuda",
    chunk_bytes: int = 64 << 20,
) -> Dict[str, Uploaded]:
    """Upload ``names`` (default: every tensor) of an open :class:`GGUFFile`.

    Returns when every copy has completed (the returned tensors are ready on
    any stream)."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"upload_gguf targets a GPU device, got {device}")
    if chunk_bytes < 4096:
        raise ValueError("chunk_bytes must be at least 4096")
    names = list(gguf.tensor_names() if names is None else names)
    chunk_bytes = min(chunk_bytes, max((gguf.tensor(n).nbytes for n in names), default=4096))
    chunk_bytes = max(4096, chunk_bytes)

    staging = [torch.empty(chunk_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    staging_np = [s.numpy() for s in staging]
    done = [None, None]  # event of the last copy out of each staging buffer
    out: Dict[str, Uploaded] = {}
    with torch.cuda.device(device):
        stream = torch.cuda.Stream(device=device)
        # device memory just allocated may have been released by work still
        # queued on the caller's stream: copy only after that work
        stream.wait_stream(torch.cuda.current_stream(device))
        raw_dev: Dict[str, torch.Tensor] = {}
        slot = 0
        for name in names:
            t = gguf.tensor(name)
            dst = torch.empty(t.nbytes, dtype=torch.uint8, device=device)
            stream.wait_stream(torch.cuda.current_stream(device))
            src = gguf.payload(name)
            for off in range(0, t.nbytes, chunk_bytes):
                n = min(chunk_bytes, t.nbytes - off)
                if done[slot] is not None:
                    done[slot].synchronize()  # the buffer's previous copy has left it
                np.copyto(staging_np[slot][:n], src[off:off + n])
                with torch.cuda.stream(stream):
                    dst[off:off + n].copy_(staging[slot][:n], non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(stream)
                done[slot] = ev
                slot ^= 1
            raw_dev[name] = dst
            del src
        stream.synchronize()

    for name, dst in raw_dev.items():
        t = gguf.tensor(name)
        ttype = t.info.ggml_type
        if ttype in FLOAT_TYPES:
            out[name] = dst.view(_TORCH_FLOAT[FLOAT_TYPES[ttype][0]]).reshape(t.shape)
        elif (base_type(t.kernel_type) in BLOCK_LAYOUTS and len(t.shape) == 2
              and t.shape[1] % BLOCK_LAYOUTS[base_type(t.kernel_type)][0] == 0):
            out[name] = GGUFQuantizedWeight(dst, t.kernel_type, t.shape)
        else:
            out[name] = dst
    return out
