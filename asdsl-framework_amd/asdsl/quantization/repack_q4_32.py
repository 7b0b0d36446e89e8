"""The reference's module name for the 20-byte preq repacker
(asdsl/quantization/repack_q4_32.py); device tensors run the HIP kernel."""

from asdsl.quantization.repack import (  # noqa: F401
    PREQ_BLOCK_SIZE as BLOCK_SIZE,
    blocks_to_flat,
    repack_asymmetric_to_q4_32_blocks,
)
