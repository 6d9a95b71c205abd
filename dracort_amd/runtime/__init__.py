"""GPU counterpart of the reference CPU executor's projection sequence."""

from dracort_amd.runtime.decode import (  # noqa: F401
    AttentionShape,
    DecodeStep,
    LayerSet,
    LlamaShape,
    layer_set_bytes,
    layer_set_from_gguf,
    synthetic_layer_set,
)
from dracort_amd.runtime.executor import (  # noqa: F401
    GPUExecutionBackend,
    GPUExecutorConfig,
    gguf_executor_config,
)
from dracort_amd.runtime.gpu_tier import GGUFGpuKernel, is_gguf_block_tensor  # noqa: F401
