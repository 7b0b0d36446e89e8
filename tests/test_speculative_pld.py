"""Prompt Lookup Decoding's draft lookup (CPU), worked by hand from the
reference's rule (asdsl/speculative/pld.py:21-45): longest n-gram first
(3, then 2), the first earlier occurrence of the context's last n tokens,
up to max_draft_k of the tokens that followed it."""

from __future__ import annotations

from asdsl.speculative.pld import PLDConfig, PromptLookupDecoder


def test_trigram_match_proposes_what_followed():
    d = PromptLookupDecoder()
    assert d.lookup([1, 2, 3, 9, 1, 2, 3]) == [9, 1, 2, 3]


def test_falls_back_to_bigram():
    d = PromptLookupDecoder()
    # last trigram (7, 5, 6) never occurred before; bigram (5, 6) did at 0
    assert d.lookup([5, 6, 7, 5, 6]) == [7, 5, 6]


def test_first_occurrence_wins_and_draft_is_capped():
    d = PromptLookupDecoder(PLDConfig(max_draft_k=2))
    ctx = [4, 8, 1, 2, 3, 4, 8, 5, 6, 4, 8]
    assert d.lookup(ctx) == [1, 2]  # (4, 8) first at 0 -> 1, 2, 3, ... capped at 2


def test_no_match_short_context_and_tail_only():
    d = PromptLookupDecoder()
    assert d.lookup([]) == [] and d.lookup([7]) == []
    assert d.lookup([1, 2, 3, 4, 5]) == []
    # the tail itself is not an earlier occurrence
    assert d.lookup([3, 3]) == []
    assert d.lookup([3, 3, 3]) == [3]  # (3, 3) at 0 is followed by one token


def test_longer_ngram_preferred_over_earlier_bigram():
    d = PromptLookupDecoder()
    ctx = [2, 3, 7, 1, 2, 3, 8, 1, 2, 3]
    # trigram (1, 2, 3) first at 3 -> 8, 1, 2, 3; the bigram (2, 3) at 0 would give 7, ...
    assert d.lookup(ctx) == [8, 1, 2, 3]
