"""I/O helpers (GGUF weight loading), as the reference's asdsl/io package."""

from asdsl.io.gguf_loader import (
    GGML_TYPE_NAMES,
    GGUF_TO_ASDSL,
    logical_shape,
    read_gguf_tensors,
    row_bytes_for_type,
)

__all__ = [
    "GGUF_TO_ASDSL",
    "GGML_TYPE_NAMES",
    "logical_shape",
    "read_gguf_tensors",
    "row_bytes_for_type",
]
