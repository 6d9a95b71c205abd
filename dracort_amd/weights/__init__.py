"""Moving GGUF weights from a file into HBM in their native block layout."""

from dracort_amd.weights.upload import upload_gguf  # noqa: F401

__all__ = ["upload_gguf"]
