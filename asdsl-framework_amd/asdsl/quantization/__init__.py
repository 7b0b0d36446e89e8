"""Weight formats consumed by the Q4 GEMV kernels (quantizer + repackers)."""
