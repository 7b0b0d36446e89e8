"""The bridge functions keep the reference's signatures
(asdsl/inference/unified_bridge.py: build_unified_engine 137,
get_or_build_unified_engine 304, reset_unified_session 338,
unified_forward_token 344-350, cpp_generate 360-365, greedy_generate
396-400, pld_generate 424-429 for the arguments it shares,
pld_generate_timed 511-516, measure_verify_overhead 533-538), so a caller
switches by import."""

from __future__ import annotations

import inspect

from asdsl.inference import unified_bridge as ub

# (name, kind, default) per parameter, as the reference declares them
REFERENCE = {
    "build_unified_engine": [("store", "POSITIONAL_OR_KEYWORD", None)],
    "get_or_build_unified_engine": [("store", "POSITIONAL_OR_KEYWORD", None)],
    "reset_unified_session": [("store", "POSITIONAL_OR_KEYWORD", None)],
    "unified_forward_token": [("store", "POSITIONAL_OR_KEYWORD", None), ("token_id", "POSITIONAL_OR_KEYWORD", None),
                              ("pos", "POSITIONAL_OR_KEYWORD", None), ("need_logits", "KEYWORD_ONLY", True)],
    "cpp_generate": [("store", "POSITIONAL_OR_KEYWORD", None), ("prompt_ids", "POSITIONAL_OR_KEYWORD", None),
                     ("max_new_tokens", "POSITIONAL_OR_KEYWORD", None), ("stop_ids", "POSITIONAL_OR_KEYWORD", None)],
    "snapshot_kv": [("engine", "POSITIONAL_OR_KEYWORD", None)],
    "restore_kv": [("engine", "POSITIONAL_OR_KEYWORD", None)],
    "truncate_kv": [("engine", "POSITIONAL_OR_KEYWORD", None), ("n", "POSITIONAL_OR_KEYWORD", None)],
    "get_kv_seq_len": [("engine", "POSITIONAL_OR_KEYWORD", None)],
    "pld_generate_timed": [("store", "POSITIONAL_OR_KEYWORD", None), ("prompt_ids", "POSITIONAL_OR_KEYWORD", None),
                           ("max_new_tokens", "POSITIONAL_OR_KEYWORD", None),
                           ("max_draft_k", "POSITIONAL_OR_KEYWORD", 6)],
    "measure_verify_overhead": [("store", "POSITIONAL_OR_KEYWORD", None), ("k_values", "KEYWORD_ONLY", (2, 4, 6)),
                                ("repeats", "KEYWORD_ONLY", 5)],
}


def test_bridge_signatures_are_the_references():
    for fn, params in REFERENCE.items():
        sig = inspect.signature(getattr(ub, fn))
        got = [(p.name, p.kind.name, None if p.default is inspect.Parameter.empty else p.default)
               for p in sig.parameters.values()]
        assert got == params, (fn, got)


def test_generators_lead_with_the_references_arguments():
    """greedy_generate(store, prompt_ids, max_new_tokens) and
    pld_generate(store, prompt_ids, max_new_tokens, max_draft_k=...): the
    reference's leading arguments (a store; here also an engine), then
    keyword options of this build."""
    g = list(inspect.signature(ub.greedy_generate).parameters)
    p = list(inspect.signature(ub.pld_generate).parameters)
    assert g[:3] == ["store", "prompt_ids", "max_new_tokens"]
    assert p[:4] == ["store", "prompt_ids", "max_new_tokens", "max_draft_k"]


def test_switches_read_as_the_reference(monkeypatch):
    """ASDSL_C01: set and not starting with '0' (unified_engine.cpp:120-123);
    ASDSL_C03: starting with '1' (engine_flags.hpp:18-24)."""
    for v, on in (("1", True), ("yes", True), ("0", False), ("", False)):
        monkeypatch.setenv("ASDSL_C01", v)
        assert ub._c01_enabled() is on
    for v, on in (("1", True), ("true", False), ("0", False)):
        monkeypatch.setenv("ASDSL_C03", v)
        assert ub._c03_enabled() is on
