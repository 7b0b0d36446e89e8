"""HIP parity for the multi-token verify pass (asdsl_decode_verify), the KV
snapshot / restore / truncate semantics and Prompt Lookup Decoding.

Bars (the decode step's: logits within 1e-3 relative L2 with top-1
agreement): every verify column has the oracle's greedy token (the oracle's
serial decode step at that position is the reference's serial fallback,
unified_engine.cpp:1774-1789) and logits within 1e-3 relative L2 of it in
at least three columns of four, all within 5e-2; the K/V rows it writes
equal the oracle's to one fp16 ulp (layers after one whose input rounded an
activation level the other way: 5e-2).  The default pass equals the
single-token step bit for bit; the MFMA form is held to 1e-5 in three
columns of four against it.  PLD returns exactly the greedy tokens.  (The stage-by-stage bars hold at full size in
test_gpu_decode_full.py: every kernel within 1e-3 of the oracle fed the
oracle's own input.)

Why not 1e-3 in every column: every GEMV quantizes its fp32 input to int8
per group, so two implementations whose fp32 sums differ by ~1e-7 (another
summation order) sometimes round one element to the neighbouring level,
which moves that GEMV's output by ~5e-4 and the logits by up to ~1e-2.
The single-token decode step shows the same against the oracle (measured at
ctx 300 over 16 positions: 2 columns at 2.5e-3 and 8.3e-3, the rest ~2e-7,
every greedy token equal).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import decode as od
from conftest import rel_l2

pytestmark = pytest.mark.gpu

# measured: 29 of 30 columns at 2e-7; one at 8.3e-3 (ctx 300, 16 columns: the
# single-token step's own int8 flip, which the pass reproduces bit for bit)
TIGHT_SHARE = 0.75
LOOSE = 5e-2


def _check_columns(errs, tight, label=None):
    """errs: per-column relative L2 errors (one JSON line of them, with
    label, to the file ASDSL_DECODE_PARITY_LOG names, if set)."""
    import json
    import os

    path = os.environ.get("ASDSL_DECODE_PARITY_LOG")
    if path and label is not None:
        with open(path, "a") as f:
            f.write(json.dumps({"test": "verify_columns", **label, "errs": [float(e) for e in errs]}) + "\n")
    errs = np.asarray(errs)
    assert np.all(errs < LOOSE), errs
    assert np.mean(errs < tight) >= TIGHT_SHARE, errs


def _host(t):
    return t.cpu().numpy()


def _engine(seed, n_layers=1, vocab=4096, max_seq=512):
    from asdsl.engine import DecodeConfig, DecodeEngine

    return DecodeEngine.synthetic(DecodeConfig(n_layers=n_layers, vocab=vocab, max_seq=max_seq), seed=seed)


def _oracle_model(eng):
    c = eng.cfg
    layers = [{n: (_host(L[n][0]), _host(L[n][1])) for n in ("qkv", "o", "gu", "down")} |
              {"rms_att": _host(L["rms_att"]), "rms_ffn": _host(L["rms_ffn"])} for L in eng.layers]
    return {"cfg": c, "layers": layers, "embed": _host(eng.embed), "rms_out": _host(eng.rms_out),
            "lm_meta": _host(eng.lm_meta), "lm_quant": _host(eng.lm_quant),
            "rope_cos": _host(eng.rope_cos), "rope_sin": _host(eng.rope_sin)}


@pytest.mark.parametrize("ctx,n", [(100, 1), (100, 4), (124, 9), (300, 16), (2100, 8)])
def test_verify_matches_serial_oracle(gpu, ctx, n):
    """n tokens at ctx .. ctx + n - 1 (124 + 9 crosses the 128-position
    split boundary; 300 + 16 spans five 64-position splits; at 2100 the
    combine folds 33-34 splits in three groups of 128 threads)."""
    eng = _engine(seed=ctx + n, n_layers=2 if n == 4 else 1, max_seq=512 if ctx + n <= 512 else 2240)
    eng.prefill_kv_random(ctx, seed=3)
    model = _oracle_model(eng)
    kc = [_host(L["k_cache"]) for L in eng.layers]
    vc = [_host(L["v_cache"]) for L in eng.layers]
    toks = [int(t) for t in np.random.default_rng(n).integers(0, eng.cfg.vocab, n)]
    logits = _host(eng.forward_batch_all_logits(toks, ctx))
    nxt = eng.verify_next_tokens()
    assert logits.shape == (n, eng.cfg.vocab) and eng.get_kv_seq_len() == ctx + n
    errs = []
    for c, t in enumerate(toks):
        want, want_next = od.decode_step(model, t, ctx + c, kc, vc)
        errs.append(rel_l2(logits[c], want))
        assert nxt[c] == want_next == od.argmax_first(logits[c]), c
    _check_columns(errs, 1e-3, {"vs": "oracle", "ctx": ctx, "n": n})
    for li, L in enumerate(eng.layers):
        gk, gv = _host(L["k_cache"]), _host(L["v_cache"])
        sl = slice(ctx, ctx + n)
        for got, want in ((gk, kc[li]), (gv, vc[li])):
            g32, w32 = got[:, sl].astype(np.float32), want[:, sl].astype(np.float32)
            if li == 0 or max(errs) < 1e-3:  # fp16 of GEMV outputs that differ in the last fp32 bits: one ulp
                np.testing.assert_allclose(g32, w32, rtol=1e-3, atol=1e-3)
            else:  # fed by a layer whose input had an activation level rounded the other way
                assert rel_l2(g32.ravel(), w32.ravel()) < 5e-2, li
        assert np.array_equal(gk[:, :ctx], kc[li][:, :ctx]) and not gk[:, ctx + n:].any()


@pytest.mark.parametrize("form", ["mfma"])
def test_verify_matches_single_token_steps(gpu, form, monkeypatch):
    """The batched pass with the projections as MFMA batched GEMVs
    (ASDSL_HIP_VERIFY_MFMA=1) against the engine's own single-token step at
    the same positions (K/V rolled back in between): 1e-5, same tokens.  The
    default form is bit for bit the single-token step
    (test_verify_is_the_single_token_step_bit_for_bit)."""
    monkeypatch.setenv("ASDSL_HIP_VERIFY_MFMA", "1")
    eng = _engine(seed=7)
    eng.prefill_kv_random(200, seed=1)
    toks = [11, 22, 33, 44, 55, 66, 77, 88]
    eng.snapshot_kv()
    batched = _host(eng.forward_batch_all_logits(toks, 200))
    bnext = eng.verify_next_tokens()
    eng.restore_kv()
    errs = []
    for c, t in enumerate(toks):
        single = _host(eng.forward_token(t, 200 + c))
        errs.append(rel_l2(batched[c], single))
        assert bnext[c] == eng.next_token(), c
    _check_columns(errs, 1e-5, {"vs": "single_token_" + form, "ctx": 200, "n": len(toks)})


def test_snapshot_restore_truncate(gpu):
    import torch

    eng = _engine(seed=2, n_layers=2, max_seq=256)
    eng.prefill_kv_random(50, seed=9)
    before = [L["k_cache"].clone() for L in eng.layers]
    eng.snapshot_kv()
    eng.forward_batch_all_logits([1, 2, 3, 4, 5], 50)
    assert eng.get_kv_seq_len() == 55 and all(L["k_cache"][:, 50:55].abs().sum() > 0 for L in eng.layers)
    eng.restore_kv()
    torch.cuda.synchronize()
    assert eng.get_kv_seq_len() == 50 and int(eng.pos.item()) == 50
    for L, b in zip(eng.layers, before):
        assert torch.equal(L["k_cache"], b) and not L["v_cache"][:, 50:].any()
    eng.restore_kv()  # empty stack: no-op
    assert eng.get_kv_seq_len() == 50
    eng.truncate_kv(20)
    assert eng.get_kv_seq_len() == 20 and all(not L["k_cache"][:, 20:].any() for L in eng.layers)
    assert all(torch.equal(L["k_cache"][:, :20], b[:, :20]) for L, b in zip(eng.layers, before))
    eng.truncate_kv(10 ** 6)  # clamps to max_seq, zeroes nothing
    assert eng.get_kv_seq_len() == 256
    eng.reset_session()
    assert eng.get_kv_seq_len() == 0 and all(not L["k_cache"].any() for L in eng.layers)
    with pytest.raises(ValueError):
        eng.forward_batch_all_logits(list(range(17)), 0)
    with pytest.raises(ValueError):
        eng.forward_batch_all_logits([1, 2], 255)


class _ListDraft:
    """Drafts tokens[len(context):] of a fixed sequence (greedy decoding's
    own continuation: every draft is accepted), or with every other drafted
    token replaced (rejections and corrections)."""

    def __init__(self, seq, k, corrupt=False):
        self.seq, self.k, self.corrupt = seq, k, corrupt

    def lookup(self, context):
        d = list(self.seq[len(context):len(context) + self.k])
        if self.corrupt:
            d = [t if i % 2 == 0 else (t + 1) % 4096 for i, t in enumerate(d)]
        return d


def _assert_greedy_up_to_ties(eng, got, want):
    """got equals want, or first differs where greedy's own step has got's
    token within 2 % of the largest |logit| of the top logit (a near-tie
    that the batched pass's rounding can turn)."""
    i = next((k for k, (a, b) in enumerate(zip(got, want)) if a != b), None)
    if i is None:
        assert got == want
        return
    eng.reset_session()
    for p, t in enumerate(want[:i]):
        logits = eng.forward_token(t, p)
    lg = _host(logits)
    assert lg[got[i]] >= lg.max() - 0.02 * np.abs(lg).max(), (i, float(lg.max()), float(lg[got[i]]))


@pytest.mark.parametrize("rerun", [True, False])
@pytest.mark.parametrize("drafter", ["lookup", "greedy", "corrupt"])
def test_pld_generate_is_greedy(gpu, rerun, drafter):
    """Prompt Lookup Decoding with the prompt-lookup drafter on a repetitive
    prompt, a drafter proposing greedy's own continuation (drafts accepted)
    and one proposing it with every other token wrong (rejections,
    corrections).  With the reference's serial re-run the tokens are exactly
    serial greedy decoding's; keeping the verify pass's K/V and argmax they
    are greedy's up to a near-tie the batched pass's rounding turns."""
    from asdsl.inference.unified_bridge import greedy_generate, pld_generate

    eng = _engine(seed=5, vocab=4096, max_seq=256)
    prompt = [5, 17, 42, 99, 5, 17, 42, 99, 5, 17]
    want = greedy_generate(eng, prompt, 40)
    dec = None if drafter == "lookup" else _ListDraft(want, 6, corrupt=drafter == "corrupt")
    stats = {}
    got = pld_generate(eng, prompt, 40, max_draft_k=6, stats=stats, rerun=rerun, decoder=dec)
    if rerun:
        assert got == want
    else:
        _assert_greedy_up_to_ties(eng, got, want)
    if drafter != "lookup":
        assert stats["verify_passes"] >= 1 and stats["accepted"] >= 1
    if drafter == "greedy" and rerun:  # (without the re-run, a turned near-tie ends the drafter's matches)
        assert stats["accepted"] >= stats["drafted"] // 2


@pytest.mark.parametrize("rerun", [True, False])
def test_pld_stops_before_end_of_sequence(gpu, rerun):
    """An end-of-sequence id that greedy decoding produces mid-way (taken
    from an unbounded run): greedy stops before it and so does PLD, whether
    it comes from the draft, the correction or a serial step."""
    from asdsl.inference.unified_bridge import greedy_generate, pld_generate

    eng = _engine(seed=5, vocab=4096, max_seq=256)
    prompt = [5, 17, 42, 99, 5, 17, 42, 99, 5, 17]
    free = greedy_generate(eng, prompt, 40, eos=())
    gen = free[len(prompt):]
    stop = gen[12]
    want = greedy_generate(eng, prompt, 40, eos=(stop,))
    assert stop not in want[len(prompt):] and len(want) < len(free)
    got = pld_generate(eng, prompt, 40, max_draft_k=6, eos=(stop,), rerun=rerun)
    if rerun:
        assert got == want
    else:
        _assert_greedy_up_to_ties(eng, got, want)
    assert stop not in got[len(prompt):]


@pytest.mark.parametrize("rerun", [True, False])
def test_pld_near_the_end_of_the_cache(gpu, rerun):
    """Generation up to the last cache position: drafts are cut at the
    cache's end (the verify pass would refuse positions past it), and the
    tokens are greedy decoding's."""
    from asdsl.inference.unified_bridge import greedy_generate, pld_generate

    eng = _engine(seed=6, vocab=4096, max_seq=64)
    prompt = [7, 8, 9, 10, 7, 8, 9, 10, 7, 8]
    n = 64 - len(prompt)
    want = greedy_generate(eng, prompt, n, eos=())
    got = pld_generate(eng, prompt, n, max_draft_k=8, eos=(), rerun=rerun, decoder=_ListDraft(want, 8))
    assert len(got) == 64
    if rerun:
        assert got == want
    else:
        _assert_greedy_up_to_ties(eng, got, want)


def test_reference_kv_length_cases(gpu):
    """The reference's tests/test_unified_kv_snapshot.py and
    test_unified_kv_truncate.py on this engine (their draft tokens run as
    ordinary steps: the layer-skipping draft mode is not part of this path)."""
    from asdsl.inference.unified_bridge import get_kv_seq_len, restore_kv, snapshot_kv, truncate_kv

    eng = _engine(seed=4, max_seq=64)
    eng.reset_session()
    for pos, tid in enumerate(range(10)):
        eng.forward_token(tid, pos)
    base_len = get_kv_seq_len(eng)
    assert base_len == 10
    snapshot_kv(eng)
    for k in range(3):
        eng.forward_token(100 + k, base_len + k)
    assert get_kv_seq_len(eng) == 13
    restore_kv(eng)
    assert get_kv_seq_len(eng) == base_len

    eng.reset_session()
    for pos, tid in enumerate(range(8)):
        eng.forward_token(tid, pos)
    committed = get_kv_seq_len(eng)
    snapshot_kv(eng)
    for k in range(4):
        eng.forward_token(200 + k, committed + k)
    assert get_kv_seq_len(eng) == committed + 4
    truncate_kv(eng, committed + 2)
    assert get_kv_seq_len(eng) == committed + 2


def test_columns_past_the_cache_write_nothing(gpu):
    """Through the C ABI (the Python API refuses it): a pass at pos =
    max_seq - 2 with 4 tokens.  The two columns inside the cache agree with a
    pass of just those two tokens (same greedy tokens); the two past it write
    no K/V (every write and read is guarded by its position) and get finite
    logits from a zero attention output."""
    import ctypes
    import torch
    from asdsl import _hip

    eng = _engine(seed=8, max_seq=128)
    eng.prefill_kv_random(120, seed=2)
    eng.forward_batch_all_logits([1, 2], 126)  # allocates the pass buffers; the two in-cache columns
    want = _host(eng._verify["logits"][:2]).copy()
    eng.truncate_kv(126)
    before = [(_host(L["k_cache"]).copy(), _host(L["v_cache"]).copy()) for L in eng.layers]
    v = eng._verify
    v["tokens"][:4].copy_(torch.tensor([1, 2, 3, 4], dtype=torch.int32))
    eng.pos.fill_(126)
    _hip.check(_hip.LIB.asdsl_decode_verify(ctypes.byref(eng._model), _hip.ptr(v["tokens"]), 4, _hip.ptr(eng.pos),
                                            _hip.ptr(v["logits"]), _hip.ptr(v["next"]), _hip.ptr(v["work"]),
                                            _hip.stream_handle()), "asdsl_decode_verify")
    torch.cuda.synchronize()
    got = _host(v["logits"][:4])
    assert np.all(np.isfinite(got))
    for c in range(2):  # the same columns through other batched kernels (4 columns, not 2)
        assert rel_l2(got[c], want[c]) < LOOSE and od.argmax_first(got[c]) == od.argmax_first(want[c])
    for L, (k0, v0) in zip(eng.layers, before):
        k1, v1 = _host(L["k_cache"]), _host(L["v_cache"])
        assert np.array_equal(k1[:, :126], k0[:, :126]) and np.array_equal(v1[:, :126], v0[:, :126])
        assert k1[:, 126:].any() and v1[:, 126:].any()  # rows 126, 127 written by the in-cache columns


def _bits_case(eng, ctx, toks):
    """The verify pass of toks at ctx, then (K/V rolled back) the engine's
    single-token steps at the same positions: logits, greedy tokens and the
    K/V rows each writes, bit for bit."""
    import torch

    n = len(toks)
    eng.snapshot_kv()
    batched = eng.forward_batch_all_logits(toks, ctx).clone()
    bnext = eng.verify_next_tokens()
    kv_b = [(L["k_cache"][:, ctx:ctx + n].clone(), L["v_cache"][:, ctx:ctx + n].clone()) for L in eng.layers]
    if eng.kv_int8:
        sc_b = [(L["k_scale"][:, ctx:ctx + n].clone(), L["v_scale"][:, ctx:ctx + n].clone()) for L in eng.layers]
    eng.restore_kv()
    for c, t in enumerate(toks):
        single = eng.forward_token(t, ctx + c)
        assert torch.equal(batched[c], single), (ctx, c, rel_l2(_host(batched[c]), _host(single)))
        assert bnext[c] == eng.next_token(), (ctx, c)
    for li, L in enumerate(eng.layers):
        assert torch.equal(L["k_cache"][:, ctx:ctx + n], kv_b[li][0]) and \
            torch.equal(L["v_cache"][:, ctx:ctx + n], kv_b[li][1]), li
        if eng.kv_int8:
            assert torch.equal(L["k_scale"][:, ctx:ctx + n], sc_b[li][0]) and \
                torch.equal(L["v_scale"][:, ctx:ctx + n], sc_b[li][1]), li


@pytest.mark.parametrize("form", ["exact_mfma", "dot4"])
@pytest.mark.parametrize("kv", ["fp16", "int8"])
@pytest.mark.parametrize("ctx,n", [(0, 3), (200, 8), (500, 16), (1000, 5), (300, 2), (700, 4)])
def test_verify_is_the_single_token_step_bit_for_bit(gpu, kv, ctx, n, form, monkeypatch):
    """The verify pass in both exact forms, on a 2-layer model (qkv/o g32
    with K split 1 and 2, gate_up, down and the lm_head g128):
      exact_mfma: MFMA GEMVs in the single-token GEMVs' fp32 order on images
        the norm, combine and SwiGLU kernels write (the default from 4
        columns; here at every column count);
      dot4 (ASDSL_HIP_VERIFY_DOT4=1): dot4 GEMVs in the single-token launch
        shapes (the default up to 3 columns; here at every column count).
    Norms in the step's order, the attention's one-tile splits: every column
    equals the single-token step at its position bit for bit, across the
    short form (below 512: o_proj merges the splits) and the long form
    (combine kernel), 500 + 16 crossing between them."""
    from asdsl.engine import DecodeConfig, DecodeEngine

    if form == "exact_mfma":
        monkeypatch.setenv("ASDSL_HIP_VERIFY_EXACT_MFMA_MIN_N", "1")  # every column count
    else:
        monkeypatch.setenv("ASDSL_HIP_VERIFY_DOT4", "1")

    eng = DecodeEngine.synthetic(DecodeConfig(n_layers=2, vocab=4096, max_seq=1100, kv_format=kv), seed=ctx + n)
    eng.prefill_kv_random(ctx, seed=5)
    toks = [int(t) for t in np.random.default_rng(ctx).integers(0, eng.cfg.vocab, n)]
    _bits_case(eng, ctx, toks)


@pytest.mark.parametrize("ctx,n", [(200, 8), (700, 16)])
def test_verify_exact_forms_with_group_32_everywhere(gpu, ctx, n):
    """The exact MFMA form's group-32 shapes beyond qkv/o: gate_up 16384x3072
    (K split 1, 6 units per lane), down 3072x8192 (K split 4, 4 units) and
    the lm_head at group size 32; every column the single-token step bit for
    bit."""
    from asdsl.engine import DecodeConfig, DecodeEngine

    eng = DecodeEngine.synthetic(DecodeConfig(n_layers=2, vocab=4096, max_seq=1024, gs_ffn=32, gs_lm=32),
                                 seed=ctx + 3)  # 8 and 16 columns: the exact MFMA form by default
    eng.prefill_kv_random(ctx, seed=6)
    toks = [int(t) for t in np.random.default_rng(ctx + 4).integers(0, eng.cfg.vocab, n)]
    _bits_case(eng, ctx, toks)


@pytest.fixture(scope="module")
def full32(gpu):
    from asdsl.engine import DecodeConfig, DecodeEngine

    return DecodeEngine.synthetic(DecodeConfig(max_seq=1100, kv_format="int8"), seed=77)


@pytest.mark.parametrize("ctx,n", [(128, 8), (1000, 16)])
def test_verify_is_the_single_token_step_bit_for_bit_full_size(full32, ctx, n):
    """The same on the 32-layer, vocab-200064 Phi-4-shaped model (qkv/o
    preq2 g32, gate_up/down/lm_head preq2-g128, int8 KV cache)."""
    full32.prefill_kv_random(ctx, seed=ctx)
    toks = [int(t) for t in np.random.default_rng(ctx + 1).integers(0, full32.cfg.vocab, n)]
    _bits_case(full32, ctx, toks)


def test_reference_calls_replay_graphs_with_the_eager_bits(gpu, monkeypatch):
    """forward_token and forward_batch_all_logits replay a HIP graph per
    position range / token count after their first call: over a sequence of
    calls at several positions and counts the logits, tokens and K/V rows
    equal those of the same calls queued eagerly (ASDSL_ENGINE_EAGER=1),
    bit for bit; and a switch changed between calls is captured anew."""
    import torch
    from asdsl.engine import DecodeConfig, DecodeEngine

    def run(eager: bool):
        if eager:
            monkeypatch.setenv("ASDSL_ENGINE_EAGER", "1")
        else:
            monkeypatch.delenv("ASDSL_ENGINE_EAGER", raising=False)
        eng = DecodeEngine.synthetic(DecodeConfig(n_layers=2, vocab=4096, max_seq=700), seed=12)
        eng.prefill_kv_random(100, seed=3)
        out = []
        for pos, tok in ((100, 5), (101, 9), (102, 5), (300, 7), (301, 8)):
            out.append((eng.forward_token(tok, pos).clone(), eng.next_token()))
        for toks, pos in (([3, 4, 5], 302), ([6, 7, 8], 305), ([1, 2], 308), ([9, 10, 11], 310)):
            out.append((eng.forward_batch_all_logits(toks, pos).clone(), tuple(eng.verify_next_tokens())))
        monkeypatch.setenv("ASDSL_HIP_VERIFY_MFMA", "1")  # another form: its own graph
        out.append((eng.forward_batch_all_logits([1, 2, 3], 320).clone(), tuple(eng.verify_next_tokens())))
        monkeypatch.delenv("ASDSL_HIP_VERIFY_MFMA")
        out.append((eng.forward_batch_all_logits([1, 2, 3], 320).clone(), tuple(eng.verify_next_tokens())))
        kv = [(L["k_cache"][:, :330].clone(), L["v_cache"][:, :330].clone()) for L in eng.layers]
        graphs = len(eng._call_graphs)
        return out, kv, graphs

    (oe, kve, ge), (og, kvg, gg) = run(True), run(False)
    assert ge == 0 and gg == 5  # two position ranges, counts 3 and 2, 3 again under the switch
    for (a, ta), (b, tb) in zip(oe, og):
        assert torch.equal(a, b) and ta == tb
    for (ka, va), (kb, vb) in zip(kve, kvg):
        assert torch.equal(ka, kb) and torch.equal(va, vb)
    mf, ex = og[-2][0], og[-1][0]  # the MFMA form: the same columns to fp32 rounding
    assert rel_l2(_host(mf), _host(ex)) < LOOSE


@pytest.mark.parametrize("kv", ["fp16", "int8"])
def test_prefill_is_forward_token_on_each_token(gpu, kv):
    """DecodeEngine.prefill runs a prompt as verify passes of up to 16
    tokens: K/V rows, logits of the last token, device token, position and
    KV length as forward_token on each prompt token in turn leaves them, bit
    for bit, for prompts of 1 to 40 tokens (single step, a 2-token pass, 16,
    16 + 1 single step, 16 + 16 + 8)."""
    import torch
    from asdsl.engine import DecodeConfig, DecodeEngine

    eng = DecodeEngine.synthetic(DecodeConfig(n_layers=2, vocab=4096, max_seq=256, kv_format=kv), seed=21)
    rng = np.random.default_rng(22)
    for plen in (1, 2, 16, 17, 40):
        prompt = [int(t) for t in rng.integers(0, eng.cfg.vocab, plen)]
        states = []
        for batched in (True, False):
            eng.reset_session()
            if batched:
                eng.prefill(prompt)
            else:
                for i, t in enumerate(prompt):
                    eng.forward_token(t, i)
            states.append((eng.logits.clone(), eng.next_token(), int(eng.pos.item()), eng._host_pos,
                           eng.get_kv_seq_len(),
                           [(L["k_cache"].clone(), L["v_cache"].clone()) for L in eng.layers]))
        (la, ta, pa, ha, ka, kva), (lb, tb, pb, hb, kb, kvb) = states
        assert torch.equal(la, lb) and (ta, pa, ha, ka) == (tb, pb, hb, kb) == (ta, plen, plen, plen), plen
        for (k1, v1), (k2, v2) in zip(kva, kvb):
            assert torch.equal(k1, k2) and torch.equal(v1, v2), plen