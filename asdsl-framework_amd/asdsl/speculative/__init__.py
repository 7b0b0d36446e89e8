"""Speculative decoding drafts (host side) for the batched verify pass."""
