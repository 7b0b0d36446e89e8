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
therefore exactly those of serial greedy decoding.  rerun=False instead
keeps the verify pass's K/V and argmax (no serial re-run).
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
                 eos=PHI4_EOS, stats: dict | None = None, rerun: bool = True, decoder: Any = None) -> list[int]:
    """Prompt Lookup Decoding with a batched verify (pld_generate,
    unified_bridge.py:424-508).  ``stats`` (optional) receives the number of
    verify passes, drafted and accepted tokens, and committed tokens
    withdrawn because the serial step disagreed.

    rerun=True, the reference's loop: after the verify pass the KV cache is
    rolled back and the committed tokens re-run one at a time; returns the
    tokens of greedy_generate.  rerun=False keeps the verify pass's K/V rows
    of the accepted tokens and takes the next token from its argmax (no
    serial re-run): one pass per draft instead of one step per token, equal
    to greedy decoding up to the fp32 rounding of the batched pass (a
    near-tie argmax can go the other way).

    Unlike the reference, the draft is looked up on the context ending with
    cur (the reference looks it up without cur, so its first draft token
    guesses cur's own slot while it is checked against the token after cur,
    and a periodic sequence has nothing accepted), no end-of-sequence token
    is committed (greedy stops before it), and a draft never runs past the
    KV cache (it is cut at max_seq - position).  The tokens returned are the
    same either way; only the acceptance differs.  ``decoder`` replaces the prompt-lookup drafter (any
    object with ``lookup(tokens) -> list[int]``)."""
    engine.reset_session()
    eos = set(eos)
    if decoder is None:
        decoder = PromptLookupDecoder(PLDConfig(max_draft_k=max_draft_k))
    tokens = [int(t) for t in prompt_ids]
    prompt_len = len(tokens)
    max_seq = int(engine.cfg.max_seq)
    counts = {"verify_passes": 0, "drafted": 0, "accepted": 0, "withdrawn": 0}
    for i, t in enumerate(tokens):
        engine.forward_token(t, i)
    pos = len(tokens)
    cur = engine.next_token()

    def room() -> int:
        return max_new_tokens - (len(tokens) - prompt_len)

    while room() > 0:
        if cur in eos:
            break
        start = pos
        # drafts for the tokens after cur: the lookup context ends with cur
        draft = decoder.lookup(tokens + [cur])[:max(0, min(max_draft_k, max_seq - start))]
        if not draft:
            tokens.append(cur)
            engine.forward_token(cur, start)
            pos = start + 1
            cur = engine.next_token()
            continue
        verify = [cur] + draft[:-1]
        if rerun:
            snapshot_kv(engine)
        engine.forward_batch_all_logits(verify, start)
        ref = engine.verify_next_tokens()
        if rerun:
            restore_kv(engine)
        accepted = 0
        for i, d in enumerate(draft):
            if ref[i] != d:
                break
            accepted += 1
        counts["verify_passes"] += 1
        counts["drafted"] += len(draft)
        counts["accepted"] += accepted
        if rerun:
            pending = [cur] + draft[:accepted]
            if accepted < len(draft):
                pending.append(ref[accepted])  # the correction
        else:
            # columns 0..a hold committed inputs; the token after them is
            # column a's argmax (draft[a] itself when every draft matched)
            a = min(accepted, len(draft) - 1)
            pending = [cur] + draft[:a]
            nxt = ref[a]
        commit = []
        for t in pending:
            if room() - len(commit) <= 0 or int(t) in eos:
                break
            commit.append(int(t))
        if not commit:
            break
        tokens.extend(commit)
        if rerun:
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
            cur = engine.next_token()  # an end-of-sequence token here ends the loop, as in greedy
        else:
            pos = start + len(commit)
            truncate_kv(engine, pos)  # drop the K/V rows of rejected drafts
            if len(commit) < len(pending):
                break  # cut by max_new_tokens or an end-of-sequence token
            cur = nxt
    if stats is not None:
        stats.update(counts)
    return tokens
