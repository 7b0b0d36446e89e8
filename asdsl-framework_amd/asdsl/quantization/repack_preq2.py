"""The reference's module name for the preq -> preq2 repacker
(asdsl/quantization/repack_preq2.py); device tensors run the HIP kernel."""

from asdsl.quantization.repack import (  # noqa: F401
    PREQ2_META_BYTES,
    PREQ2_ROW_BAND,
    meta_to_flat,
    preq2_flat_sizes,
    quant_to_flat,
    repack_preq_blocks_to_preq2,
)

PREQ2_GROUP_QUANT_BYTES = 64
