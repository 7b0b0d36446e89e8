"""Generation drivers over the GPU decode engine."""
