"""Prompt Lookup Decoding: draft tokens from an earlier occurrence of the
context's last n-gram, no draft model (asdsl/speculative/pld.py:8-45).

The lookup tries n-gram lengths from ``max_ngram`` down to ``min_ngram``; for
each it scans the context left to right for the first earlier occurrence of
the last n tokens that has at least one token after it, and proposes up to
``max_draft_k`` tokens that followed it.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass
class PLDConfig:
    max_ngram: int = 3
    min_ngram: int = 2
    max_draft_k: int = 6


class PromptLookupDecoder:
    def __init__(self, config: PLDConfig | None = None) -> None:
        self.config = config or PLDConfig()

    def lookup(self, context: list[int]) -> list[int]:
        """Draft token ids, possibly empty."""
        cfg = self.config
        L = len(context)
        if L < cfg.min_ngram:
            return []
        ctx = [int(t) for t in context]
        for n in range(cfg.max_ngram, cfg.min_ngram - 1, -1):
            if n > L:
                continue
            tail = ctx[L - n:]
            # earlier starts only (i + n < L keeps the occurrence off the tail
            # itself and leaves at least one following token)
            for i in range(L - n):
                if ctx[i:i + n] == tail:
                    follow = ctx[i + n:i + n + cfg.max_draft_k]
                    if follow:
                        return follow
        return []
