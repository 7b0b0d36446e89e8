"""The reference's bridge (asdsl/inference/unified_bridge.py) over
``asdsl.engine.DecodeEngine``: building the engine from a loaded weight
store (build_unified_engine 137-301, get_or_build_unified_engine 304-335),
single steps (unified_forward_token 344-357), the whole-generation loop
(cpp_generate 360-382), session reset (reset_unified_session 338-341), the
KV helpers (65-83), serial greedy decoding (greedy_generate 396-421),
lossless Prompt Lookup Decoding with a batched verify (pld_generate 424-508,
pld_generate_timed 511-530) and the verify-cost probe
(measure_verify_overhead 533-573).  Each takes what the reference's takes --
a WeightStore -- or, here also, a DecodeEngine directly.

A store is duck-typed on the attributes the reference reads from
experiments/phi4_cpu_run.py's WeightStore: ``group_size``; per (layer,
projection name) the preq blocks ``_preq_blocks_np`` (20-byte Q4_32 at group
size 32, 66-byte Q4_128 at 128), the preq2 operands ``_preq2_meta_np`` /
``_preq2_quant_np`` once ``_preq2_built``, the C0.1/C0.3 group-128 blocks
``_preq_gs128_np``; ``_norm_np`` or ``get_norm(layer, name)``;
``embed_f16`` (the tied output projection too); ``final_norm``;
``lm_head`` (only its row count, the vocabulary).  The model shape is
Phi-4's unless the store carries a ``decode_config`` (asdsl.engine.DecodeConfig);
the KV cache holds 2048 positions, as the reference's engine (cfg.max_seq_len,
unified_bridge.py:180).  The switches are the reference's environment:
ASDSL_C01 (gate_up/down from the group-128 blocks), ASDSL_C03 (qkv/o too),
ASDSL_LMHEAD_GS (the lm_head group size, default the store's), ASDSL_PREQ2,
PHI4_NO_LMHEAD_PREQ2_CACHE, ASDSL_IGNORE_EOS.

pld_generate verifies a draft in one multi-token pass (the verify columns'
greedy tokens come from the GPU), then, like the reference, rolls the KV
cache back and re-runs the committed tokens one at a time.  Each re-run
step's own argmax is checked against the next committed token, and the
commit stops at the first disagreement (the serial token then comes next),
so the returned tokens are exactly those of serial greedy decoding whatever
the pass computes.  rerun=False instead keeps the verify pass's K/V and
argmax (no serial re-run).  The default pass is the single-token step bit
for bit below 2048 positions, so that is lossless too; with the MFMA form
(ASDSL_HIP_VERIFY_MFMA=1) the pass follows the step only to fp32 rounding,
which int8 activation quantization can turn into a different argmax where
two logits are close.
"""

from __future__ import annotations

import os
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

from asdsl.speculative.pld import PLDConfig, PromptLookupDecoder

PHI4_EOS = (199999, 200020)
ENGINE_MAX_SEQ = 2048  # the reference bridge's cfg.max_seq_len


def _c01_enabled() -> bool:
    v = os.environ.get("ASDSL_C01", "")  # unified_engine.cpp:120-123: set, first character not '0'
    return bool(v) and v[0] != "0"


def _c03_enabled() -> bool:
    return os.environ.get("ASDSL_C03", "")[:1] == "1"  # engine_flags.hpp:18-24


def _env_yes(name: str, default: str = "0") -> bool:
    return os.environ.get(name, default).strip().lower() in ("1", "true", "yes")


def _preq2_on() -> bool:
    return os.environ.get("ASDSL_PREQ2", "0").strip().lower() not in ("0", "false", "no")


def _lm_head_gs(store: Any) -> int:
    return int(os.environ.get("ASDSL_LMHEAD_GS", str(int(store.group_size))))


def _lmhead_cache_path(store: Any) -> Path | None:
    """The reference's lm_head cache file beside the store's weight cache
    (lmhead_preq2_cache.py:58-68) when the store names one; None otherwise
    (the reference then derives a model-directory digest, which is the
    loader's business)."""
    wc = getattr(store, "_weight_cache_path", None)
    if wc is None:
        return None
    wc = Path(wc)
    digest = wc.stem.replace("phi4_cpu_", "")
    return wc.parent / f"phi4_lmhead_preq2_{digest}_gs{_lm_head_gs(store)}.safetensors"


def _engine_of(x: Any):
    """A DecodeEngine as it is, or the store's engine (built on first use)."""
    from asdsl.engine import DecodeEngine

    return x if isinstance(x, DecodeEngine) else get_or_build_unified_engine(x)


def build_unified_engine(store: Any):
    """A DecodeEngine from a loaded weight store (build_unified_engine,
    unified_bridge.py:137-301): the projections' preq2 operands (the store's
    own when built, else repacked on the device from its preq blocks; the
    group-128 blocks for gate_up/down under ASDSL_C01 and for qkv/o under
    ASDSL_C03), the norms, the fp16 embedding, and the lm_head -- from the
    store's lm_head preq2 cache when ASDSL_PREQ2 is on, the lm_head group
    size is 32 and the cache file matches, else the tied embedding
    quantized as the reference's engine does at load
    (asdsl.quantization.lm_head; the bridge passes the embedding as the
    output projection, unified_bridge.py:211-222), and then written to that
    cache as the reference does (290-299)."""
    import torch
    from dataclasses import replace

    from asdsl import _hip
    from asdsl.engine import DecodeConfig, DecodeEngine
    from asdsl.quantization.lm_head import quantize_output_projection
    from asdsl.quantization.preq_cache import preq2_from_preq_blocks

    dev = _hip.device()
    gs = int(store.group_size)
    if gs not in (32, 128):
        raise ValueError(f"build_unified_engine: store group_size must be 32 or 128, got {gs}")
    given = getattr(store, "decode_config", None)
    cfg = given if given is not None else DecodeConfig(max_seq=ENGINE_MAX_SEQ)
    embed = store.embed_f16
    embed = (embed if isinstance(embed, torch.Tensor) else torch.from_numpy(np.asarray(embed))).to(dev)
    embed = embed.to(torch.float16).contiguous()
    lm = getattr(store, "lm_head", None)
    vocab = int(lm.shape[0]) if lm is not None else int(embed.shape[0])
    g128 = getattr(store, "_preq_gs128_np", None) or {}

    def has128(names):
        return all((i, n) in g128 for i in range(cfg.n_layers) for n in names)

    gs_ffn = 128 if _c01_enabled() and has128(("gate_up_proj", "down_proj")) else gs
    gs_attn = 128 if _c03_enabled() and has128(("qkv_proj", "o_proj")) else gs
    lm_gs = _lm_head_gs(store)
    cfg = replace(cfg, vocab=vocab, gs_attn=gs_attn, gs_ffn=gs_ffn, gs_lm=lm_gs)
    if embed.dim() != 2 or embed.shape[1] != cfg.hidden:
        raise ValueError(f"build_unified_engine: embedding {tuple(embed.shape)} does not match hidden {cfg.hidden}")
    shapes = {"qkv_proj": (cfg.qkv_dim, cfg.hidden, gs_attn), "o_proj": (cfg.hidden, cfg.hidden, gs_attn),
              "gate_up_proj": (2 * cfg.ffn, cfg.hidden, gs_ffn), "down_proj": (cfg.hidden, cfg.ffn, gs_ffn)}
    short = {"qkv_proj": "qkv", "o_proj": "o", "gate_up_proj": "gu", "down_proj": "down"}
    preq2_built = bool(getattr(store, "_preq2_built", False))
    meta_np = getattr(store, "_preq2_meta_np", None) or {}
    quant_np = getattr(store, "_preq2_quant_np", None) or {}
    blocks_np = getattr(store, "_preq_blocks_np", None) or {}
    norm_np = getattr(store, "_norm_np", None) or {}

    def up(a, dtype=torch.uint8):
        t = a.detach() if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))
        return t.to(dev).to(dtype).contiguous().reshape(-1)

    def norm(i, name):
        w = norm_np.get((i, name))
        if w is None:
            w = store.get_norm(i, name)
        return up(w, torch.float32)

    layers = []
    for i in range(cfg.n_layers):
        L = {}
        for name, (rows, cols, pgs) in shapes.items():
            key = (i, name)
            if pgs == 128 and key in g128:
                L[short[name]] = preq2_from_preq_blocks(up(g128[key]), rows, cols, 128)
            elif pgs == 32 and preq2_built and key in meta_np and key in quant_np:
                L[short[name]] = (up(meta_np[key]), up(quant_np[key]))
            elif key in blocks_np:
                L[short[name]] = preq2_from_preq_blocks(up(blocks_np[key]), rows, cols, pgs)
            else:
                raise ValueError(f"build_unified_engine: no weights for layer {i} {name}")
        L["rms_att"] = norm(i, "input_layernorm")
        L["rms_ffn"] = norm(i, "post_attention_layernorm")
        layers.append(L)
    rms_out = up(store.final_norm, torch.float32)

    lm_meta = lm_quant = None
    cache = _lmhead_cache_path(store) if _preq2_on() and lm_gs == 32 else None
    if cache is not None:
        from asdsl.quantization.lmhead_preq2_cache import try_restore_lmhead_preq2_cache

        got = try_restore_lmhead_preq2_cache(store, cache, device=dev)
        if got is not None:
            lm_meta, lm_quant = got
    if lm_meta is None:
        lm_meta, lm_quant = quantize_output_projection(embed, lm_gs)
        if cache is not None:
            from asdsl.quantization.lmhead_preq2_cache import save_lmhead_preq2_cache

            save_lmhead_preq2_cache(store, cache, lm_meta.cpu().numpy(), lm_quant.cpu().numpy())
    return DecodeEngine(cfg, layers, embed, rms_out, lm_meta, lm_quant,
                        float(getattr(store, "fatrelu_threshold", 0.0) or 0.0))


def get_or_build_unified_engine(store: Any):
    """The store's engine, built once and kept on the store
    (get_or_build_unified_engine, unified_bridge.py:304-335)."""
    eng = getattr(store, "_unified_engine", None)
    if eng is None:
        eng = build_unified_engine(store)
        store._unified_engine = eng
    return eng


def reset_unified_session(store: Any) -> None:
    """Empty KV cache (reset_unified_session, unified_bridge.py:338-341)."""
    get_or_build_unified_engine(store).reset_session()


def unified_forward_token(store: Any, token_id: int, pos: int, *, need_logits: bool = True) -> np.ndarray | None:
    """One decode step (unified_forward_token, unified_bridge.py:344-357):
    the logits as a float32 numpy array, or None with need_logits=False (the
    K/V rows are written either way; the reference's prefill body)."""
    eng = get_or_build_unified_engine(store)
    logits = eng.forward_token(int(token_id), int(pos))
    if need_logits:
        return logits.cpu().numpy().astype(np.float32, copy=False)
    return None


def cpp_generate(store: Any, prompt_ids: list[int], max_new_tokens: int,
                 stop_ids: list[int] | None = None) -> list[int]:
    """The whole generation on the device (cpp_generate, unified_bridge.py:
    360-382, over UnifiedEngine::generate, unified_engine.cpp:1717-1762):
    reset, the prompt one step each, then greedy tokens from captured step
    graphs until max_new_tokens or a stop token, which is included (the
    engine appends it, then stops).  Stop tokens default to Phi-4's; none
    with ASDSL_IGNORE_EOS.  Returns the new tokens only."""
    eng = get_or_build_unified_engine(store)
    eng.reset_session()
    stop = set() if _env_yes("ASDSL_IGNORE_EOS", "") else {int(t) for t in (stop_ids or PHI4_EOS)}
    prompt = [int(t) for t in prompt_ids]
    eng.prefill(prompt)  # as forward_token on each prompt token, in verify passes
    out: list[int] = []
    if not prompt:
        return out
    # the device keeps the token: steps run in chunks (decode_steps), each
    # read once; the engine ends as one step per token leaves it
    pending = [eng.next_token()]
    stepped = len(prompt)
    while len(out) < int(max_new_tokens):
        if not pending:
            k = min(_GREEDY_CHUNK, int(max_new_tokens) - len(out), eng.cfg.max_seq - stepped)
            if k <= 0:
                break
            pending = eng.decode_steps(k)
            stepped += k
        best = pending.pop(0)
        out.append(best)
        if best in stop or len(prompt) + len(out) > eng.cfg.max_seq:
            break
    n = len(prompt) + len(out)
    # the per-token loop steps every generated token but a final stop token
    # (or one past the cache)
    if out and (out[-1] in stop or n > eng.cfg.max_seq):
        _settle(eng, n - 1, out[-2] if len(out) > 1 else prompt[-1], stepped, out[-1])
    elif out:
        _settle(eng, n, out[-1], stepped, pending[0] if pending else None)
    return out


def snapshot_kv(engine: Any) -> None:
    engine.snapshot_kv()


def restore_kv(engine: Any) -> None:
    engine.restore_kv()


def truncate_kv(engine: Any, n: int) -> None:
    engine.truncate_kv(int(n))


def get_kv_seq_len(engine: Any) -> int:
    return int(engine.get_kv_seq_len())


def greedy_generate(store: Any, prompt_ids: list[int], max_new_tokens: int, eos=PHI4_EOS) -> list[int]:
    """Serial greedy decode: the prompt one token at a time, then the argmax
    of each step until max_new_tokens or an end-of-sequence token (which is
    not appended).  Returns prompt and new tokens.  store: a weight store or
    a DecodeEngine."""
    engine = _engine_of(store)
    engine.reset_session()
    eos = set(eos)
    tokens = [int(t) for t in prompt_ids]
    prompt_len = len(tokens)
    engine.prefill(tokens)  # as forward_token on each prompt token, in verify passes
    if not tokens:
        return tokens
    # Steps run in chunks on the device (decode_steps: one read per chunk);
    # the engine ends as the one-step-per-token loop leaves it.
    pending = [engine.next_token()]
    stepped = len(tokens)  # positions whose step has run
    stop_tok = None
    while len(tokens) - prompt_len < max_new_tokens:
        if not pending:
            k = min(_GREEDY_CHUNK, max_new_tokens - (len(tokens) - prompt_len), engine.cfg.max_seq - stepped)
            if k <= 0:
                break
            pending = engine.decode_steps(k)
            stepped += k
        cur = pending.pop(0)
        if cur in eos:
            stop_tok = cur
            break
        tokens.append(cur)
    # the per-token loop steps every position 0 .. len(tokens) - 1
    _settle(engine, len(tokens), tokens[-1], stepped, stop_tok if stop_tok is not None else
            (pending[0] if pending else None))
    return tokens


# greedy steps per device read in greedy_generate and cpp_generate
_GREEDY_CHUNK = 16


def _settle(engine: Any, n: int, last: int, stepped: int, after: int | None) -> None:
    """Leave the engine as a loop of one step per token leaves it: the steps
    of positions 0 .. n - 1 run and no other, the device token the one the
    step at n - 1 gives, the position n.  last: the token at position n - 1;
    stepped: positions whose step ran (a chunk may run past the last token
    taken); after: the token the step at n - 1 gave, when known."""
    if stepped < n:  # the last token's own step
        engine.forward_token(last, n - 1)
    elif stepped > n:  # steps past it: drop their K/V rows, restore its successor
        engine.truncate_kv(n)
        engine.token.fill_(int(after))


def pld_generate(store: Any, prompt_ids: list[int], max_new_tokens: int, max_draft_k: int = 6,
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
    object with ``lookup(tokens) -> list[int]``).  store: a weight store or a DecodeEngine."""
    engine = _engine_of(store)
    engine.reset_session()
    eos = set(eos)
    if decoder is None:
        decoder = PromptLookupDecoder(PLDConfig(max_draft_k=max_draft_k))
    tokens = [int(t) for t in prompt_ids]
    prompt_len = len(tokens)
    max_seq = int(engine.cfg.max_seq)
    counts = {"verify_passes": 0, "drafted": 0, "accepted": 0, "withdrawn": 0}
    engine.prefill(tokens)  # as forward_token on each prompt token, in verify passes
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


@dataclass
class PldResult:
    """Result of a timed generation (PldResult, unified_bridge.py:385-393)."""

    token_ids: list[int]
    prompt_len: int
    decode_tokens: int
    decode_s: float
    tokens_per_second: float


def pld_generate_timed(store: Any, prompt_ids: list[int], max_new_tokens: int, max_draft_k: int = 6) -> PldResult:
    """pld_generate with wall-clock timing (pld_generate_timed,
    unified_bridge.py:511-530)."""
    t0 = time.perf_counter()
    out = pld_generate(store, prompt_ids, max_new_tokens, max_draft_k=max_draft_k)
    decode_s = time.perf_counter() - t0
    prompt_len = len(prompt_ids)
    decode_tokens = max(0, len(out) - prompt_len)
    return PldResult(token_ids=out, prompt_len=prompt_len, decode_tokens=decode_tokens, decode_s=float(decode_s),
                     tokens_per_second=float(decode_tokens / decode_s if decode_s > 0 else 0.0))


def measure_verify_overhead(store: Any, *, k_values: tuple[int, ...] = (2, 4, 6), repeats: int = 5) -> dict:
    """Cost of a k-token verify pass against one step (measure_verify_overhead,
    unified_bridge.py:533-573): three probe tokens prefilled, then the median
    over `repeats` of one step at position 3 and of one k-column pass from
    position 3, the KV cache restored after each; host clock around each call
    with the device synchronized, ms.  Keys t_single_ms, t_verify_k{k}_ms,
    ratio_k{k}, vocab."""
    import torch

    eng = _engine_of(store)
    eng.reset_session()
    probe = [100, 200, 300, 400, 500, 600, 700, 800, 900, 1000]
    probe = [t % eng.cfg.vocab for t in probe]
    for i, tid in enumerate(probe[:3]):
        eng.forward_token(int(tid), i)
    start_pos = 3

    def timed(fn) -> float:
        ms = []
        for _ in range(repeats):
            snapshot_kv(eng)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ms.append((time.perf_counter() - t0) * 1000.0)
            restore_kv(eng)
        return float(np.median(ms))

    t_single = timed(lambda: eng.forward_token(int(probe[3]), start_pos))
    out: dict = {"t_single_ms": round(t_single, 3)}
    for k in k_values:
        toks = [int(probe[3 + j]) for j in range(k)]
        t_k = timed(lambda: eng.forward_batch_all_logits(toks, start_pos))
        out[f"t_verify_k{k}_ms"] = round(t_k, 3)
        out[f"ratio_k{k}"] = round(t_k / t_single if t_single > 0 else 0.0, 3)
    out["vocab"] = float(eng.cfg.vocab)
    return out
