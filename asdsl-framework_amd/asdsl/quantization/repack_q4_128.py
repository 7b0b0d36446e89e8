"""The reference's module name for the 66-byte Q4_128 repackers
(asdsl/quantization/repack_q4_128.py); device tensors run the HIP kernels."""

from asdsl.quantization.repack import (  # noqa: F401
    Q4_128_BLOCK_SIZE as BLOCK_SIZE,
    blocks_to_flat,
    repack_asymmetric_to_q4_128_blocks,
    repack_fp32_to_q4_128_blocks,
)

GROUP_SIZE = 128
