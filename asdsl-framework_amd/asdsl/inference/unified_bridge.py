"""Generation loops over ``asdsl.engine.DecodeEngine``, mirroring the
reference's bridge (asdsl/inference/unified_bridge.py): the KV helpers
(65-83), serial greedy decoding (greedy_generate, 396-421) and lossless
Prompt Lookup Decoding with a batched verify (pld_generate, 424-508).  The
reference's functions take a WeightStore and build or fetch its engine; these
take the engine.

pld_generate verifies a draft in one multi-token pass (the verify columns'
greedy tokens come from the GPU), then, like the reference, rolls the KV
cache back and re-runs the committed tokens one at a time.  The batched pass
follows the single-token step's arithmetic only to fp32 rounding, and int8
activation quantization can turn such a difference into a different argmax
where two logits are close; so each re-run step's own argmax is checked
against the next committed token, and the commit stops at the first
disagreement (the serial token then comes next).  The returned tokens are
therefore exactly those of serial greedy decoding.
"""

from __future__ import annotations

from typing import Any

from asdsl.speculative.pld import PLDConfig, PromptLookupDecoder

PHI4_EOS = (199999, 200020)


def snapshot_kv(engine: Any) -> None:
    engine.snapshot_kv()


def restore_kv(engine: Any) -> None:
    engine.restore_kv()


def truncate_kv(engine: Any, n: int) -> None:
    engine.truncate_kv(int(n))


def get_kv_seq_len(engine: Any) -> int:
    return int(engine.get_kv_seq_len())


def greedy_generate(engine: Any, prompt_ids: list[int], max_new_tokens: int, eos=PHI4_EOS) -> list[int]:
    """Serial greedy decode: the prompt one token at a time, then the argmax
    of each step until max_new_tokens or an end-of-sequence token."""
    engine.reset_session()
    eos = set(eos)
    tokens = [int(t) for t in prompt_ids]
    prompt_len = len(tokens)
    for i, t in enumerate(tokens):
        engine.forward_token(t, i)
    pos = len(tokens)
    while len(tokens) - prompt_len < max_new_tokens:
        cur = engine.next_token()
        if cur in eos:
            break
        tokens.append(cur)
        engine.forward_token(cur, pos)
        pos += 1
    return tokens


def pld_generate(engine: Any, prompt_ids: list[int], max_new_tokens: int, max_draft_k: int = 6,
                 eos=PHI4_EOS, stats: dict | None = None) -> list[int]:
    """Prompt Lookup Decoding with a batched verify; returns the same tokens
    as greedy_generate.  ``stats`` (optional) receives the number of verify
    passes, drafted and accepted tokens, and committed tokens withdrawn
    because the serial step disagreed."""
    engine.reset_session()
    eos = set(eos)
    decoder = PromptLookupDecoder(PLDConfig(max_draft_k=max_draft_k))
    tokens = [int(t) for t in prompt_ids]
    prompt_len = len(tokens)
    counts = {"verify_passes": 0, "drafted": 0, "accepted": 0, "withdrawn": 0}
    for i, t in enumerate(tokens):
        engine.forward_token(t, i)
    pos = len(tokens)
    while len(tokens) - prompt_len < max_new_tokens:
        cur = engine.next_token()
        if cur in eos:
            break
        start = pos
        draft = decoder.lookup(tokens)[:max_draft_k]
        if not draft:
            tokens.append(cur)
            engine.forward_token(cur, start)
            pos = start + 1
            continue
        verify = [cur] + draft[:-1]
        snapshot_kv(engine)
        engine.forward_batch_all_logits(verify, start)
        ref = engine.verify_next_tokens()
        restore_kv(engine)
        accepted = 0
        correction = None
        for i, d in enumerate(draft):
            if ref[i] == d:
                accepted += 1
            else:
                correction = ref[i]
                break
        counts["verify_passes"] += 1
        counts["drafted"] += len(draft)
        counts["accepted"] += accepted
        pending = [cur] + draft[:accepted] + ([correction] if correction is not None else [])
        commit = []
        for t in pending:
            if len(tokens) - prompt_len >= max_new_tokens:
                break
            commit.append(int(t))
            tokens.append(int(t))
        if not commit:
            break
        truncate_kv(engine, start)
        kept = 0
        for j, t in enumerate(commit):
            engine.forward_token(t, start + j)
            kept += 1
            if j + 1 < len(commit) and engine.next_token() != commit[j + 1]:
                break  # the serial step disagrees with the batched pass: its token comes next
        if kept < len(commit):
            counts["withdrawn"] += len(commit) - kept
            del tokens[len(tokens) - (len(commit) - kept):]
            commit = commit[:kept]
        pos = start + kept
        if len(tokens) - prompt_len >= max_new_tokens or any(t in eos for t in commit):
            break
    if stats is not None:
        stats.update(counts)
    return tokens
