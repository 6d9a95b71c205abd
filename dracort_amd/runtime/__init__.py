"""GPU counterpart of the reference CPU executor's projection sequence."""

from dracort_amd.runtime.decode import (  # noqa: F401
    DecodeStep,
    LayerSet,
    LlamaShape,
    layer_set_bytes,
    synthetic_layer_set,
)
from dracort_amd.runtime.gpu_tier import GGUFGpuKernel, is_gguf_block_tensor  # noqa: F401
