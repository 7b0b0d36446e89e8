"""Decode-step parity at full size: the 32-layer, vocab-200064 Phi-4-shaped
model that bench.py times (hidden 3072, FFN 8192, 24/8 heads, qkv/o preq2
g32, gate_up/down/lm_head preq2-g128, fp16 KV cache prefilled with N(0,1)),
against oracle/decode.py at contexts 128, 1024 and 4096.

Two kinds of test:

* Per layer, teacher forced (test_full_layers_teacher_forced).  At every
  step the oracle runs the whole model; then every kernel the decode step
  chains is run on the GPU for every one of the 32 layers and the lm_head,
  each fed the oracle's own input for that stage, on the real weights and
  the real KV cache at that context: the qkv GEMV with its residual +
  RMSNorm prologue, RoPE + KV write + attention, the o_proj GEMV, the
  gate_up GEMV with its prologue and SwiGLU epilogue (compared as the
  SwiGLU output), the down GEMV, and the lm_head with its norm prologue and
  argmax epilogue.  Bars: 1e-4
  relative L2 for the kernels whose int8 activation comes from the same
  fp32 input (attention, o_proj, down), 1e-3 for those that compute the
  RMSNorm themselves (one ulp of inv_rms can move an int8 level), the
  residual stream bit-exact, and the greedy token of >= 99 % of the steps.

* End to end (test_full_decode_end_to_end).  Whole decode steps on the GPU
  against the oracle, teacher forced (both get the oracle's token), each
  with its own KV cache.  This random-weight 32-layer model amplifies a
  rounding difference chaotically: one int8 activation level that two
  summation orders round differently moves the logits by ~1e-3 in the next
  layers and by ~1e-1 after 32.  The oracle against itself with the GEMV
  sums taken in float32 (oracle.gemv_preq2_fused_f32sum) shows the same
  spread, so the bar is relative to it: the GPU's median relative L2 within
  3x that of the second CPU restatement (+ 1e-3), and its greedy-token
  agreement no more than 0.25 below that restatement's.

Set ASDSL_DECODE_PARITY_LOG to a file path to get one JSON line per step.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from conftest import rel_l2

pytestmark = pytest.mark.gpu

CONTEXTS = (128, 1024, 4096)
STEPS_LAYERWISE = 16
STEPS_E2E = 16
_TOKENS: dict[int, list] = {}


def _log(rows):
    path = os.environ.get("ASDSL_DECODE_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            for r in rows:
                f.write(json.dumps(r) + "\n")


@pytest.fixture(scope="module")
def full_model(gpu):
    from asdsl.engine import DecodeConfig, DecodeEngine
    from oracle import decode as od

    eng = DecodeEngine.synthetic(DecodeConfig(max_seq=4224), seed=2024)
    return eng, od.host_model(eng)


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("ctx", CONTEXTS)
def test_full_layers_teacher_forced(full_model, ctx):
    import torch
    from asdsl import _hip
    from oracle import decode as od

    eng, model = full_model
    c = eng.cfg
    eng.prefill_kv_random(ctx, seed=ctx)
    kc = [L["k_cache"].cpu().numpy() for L in eng.layers]
    vc = [L["v_cache"].cpu().numpy() for L in eng.layers]
    s = _hip.stream_handle()
    P = _hip.ptr
    qkv = torch.empty(c.qkv_dim, device="cuda")
    att = torch.empty(c.hidden, device="cuda")
    o = torch.empty(c.hidden, device="cuda")
    hmid = torch.empty(c.hidden, device="cuda")
    gu = torch.empty(2 * c.ffn, device="cuda")
    down = torch.empty(c.hidden, device="cuda")
    logits = torch.empty(c.vocab, device="cuda")
    key = torch.zeros(1, dtype=torch.int64, device="cuda")
    work = torch.zeros(_hip.LIB.asdsl_attention_work_floats(c.n_heads, c.max_seq), device="cuda")
    dpos = torch.zeros(1, dtype=torch.int32, device="cuda")
    tok, worst, rows, agree = 1000 + ctx, {}, [], 0
    for step in range(STEPS_LAYERWISE):
        pos = ctx + step
        trace = []
        want_logits, want_next = od.decode_step(model, tok, pos, kc, vc, trace=trace)
        dpos.fill_(pos)
        for li, (L, t) in enumerate(zip(eng.layers, trace[:-1])):
            dh = _dev(t["h"])
            _hip.call("asdsl_gemv_preq2_rmsnorm", P(L["qkv"][0]), P(L["qkv"][1]), P(dh), None, P(L["rms_att"]), None,
                      P(qkv), c.qkv_dim, c.hidden, c.gs_attn, c.rms_eps, None, s)
            _hip.call("asdsl_attention_f16kv", P(_dev(t["qkv"])), P(L["k_cache"]), P(L["v_cache"]), P(eng.rope_cos),
                      P(eng.rope_sin), P(dpos), P(att), P(work), c.n_heads, c.n_kv_heads, c.head_dim, c.rotary_dim,
                      c.max_seq, s)
            _hip.call("asdsl_gemv_preq2_fused", P(L["o"][0]), P(L["o"][1]), P(_dev(t["att"])), P(o), c.hidden,
                      c.hidden, c.gs_attn, s)
            _hip.call("asdsl_gemv_preq2_rmsnorm_swiglu", P(L["gu"][0]), P(L["gu"][1]), P(dh), P(_dev(t["o"])),
                      P(L["rms_ffn"]), P(hmid), P(gu), c.ffn, c.hidden, c.gs_ffn, c.rms_eps, 0.0, s)
            _hip.call("asdsl_gemv_preq2_fused", P(L["down"][0]), P(L["down"][1]), P(_dev(t["s"])), P(down),
                      c.hidden, c.ffn, c.gs_ffn, s)
            torch.cuda.synchronize()
            errs = {"qkv": rel_l2(qkv.cpu().numpy(), t["qkv"]), "att": rel_l2(att.cpu().numpy(), t["att"]),
                    "o": rel_l2(o.cpu().numpy(), t["o"]), "gu": rel_l2(gu[: c.ffn].cpu().numpy(), t["s"]),
                    "down": rel_l2(down.cpu().numpy(), t["down"])}
            assert np.array_equal(hmid.cpu().numpy().view(np.uint32), t["h_mid"].view(np.uint32)), (pos, li)
            for k, v in errs.items():
                worst[k] = max(worst.get(k, 0.0), v)
            assert errs["att"] < 1e-4 and errs["o"] < 1e-4 and errs["down"] < 1e-4, (pos, li, errs)
            assert errs["qkv"] < 1e-3 and errs["gu"] < 1e-3, (pos, li, errs)
            # the GPU wrote its own K/V row at pos; keep the oracle's, so the
            # next step of every layer starts from identical caches
            L["k_cache"][:, pos] = torch.from_numpy(kc[li][:, pos]).cuda()
            L["v_cache"][:, pos] = torch.from_numpy(vc[li][:, pos]).cuda()
        key.zero_()
        _hip.call("asdsl_gemv_preq2_rmsnorm", P(eng.lm_meta), P(eng.lm_quant), P(_dev(trace[-1]["h"])), None,
                  P(eng.rms_out), None, P(logits), c.vocab, c.hidden, c.gs_lm, c.rms_eps, P(key), s)
        torch.cuda.synchronize()
        lm_err = rel_l2(logits.cpu().numpy(), want_logits)
        worst["lm_head"] = max(worst.get("lm_head", 0.0), lm_err)
        assert lm_err < 1e-3, (pos, lm_err)
        got_next = 0xFFFFFFFF - (int(key.item()) & 0xFFFFFFFF)
        agree += got_next == want_next
        rows.append({"test": "layerwise", "ctx": ctx, "pos": pos, "lm_head_rel_l2": lm_err,
                     "agree": got_next == want_next})
        tok = want_next
    rows.append({"test": "layerwise_worst", "ctx": ctx, **worst})
    _log(rows)
    assert agree >= 0.99 * STEPS_LAYERWISE, agree


@pytest.mark.parametrize("ctx", CONTEXTS)
def test_full_decode_end_to_end(full_model, ctx):
    import torch
    from oracle import decode as od

    eng, model = full_model
    eng.prefill_kv_random(ctx, seed=ctx + 1)
    kc = [L["k_cache"].cpu().numpy() for L in eng.layers]
    vc = [L["v_cache"].cpu().numpy() for L in eng.layers]
    kc2 = [k.copy() for k in kc]
    vc2 = [v.copy() for v in vc]
    tok = 200 + ctx
    rows = []
    for step in range(STEPS_E2E):
        pos = ctx + step
        want_logits, want_next = od.decode_step(model, tok, pos, kc, vc)
        alt_logits, alt_next = od.decode_step(model, tok, pos, kc2, vc2, gemv=oracle.gemv_preq2_fused_f32sum)
        eng.forward_token(tok, pos)
        torch.cuda.synchronize()
        rows.append({"test": "end_to_end", "ctx": ctx, "pos": pos,
                     "rel_l2": rel_l2(eng.logits.cpu().numpy(), want_logits), "agree": eng.next_token() == want_next,
                     "f32sum_rel_l2": rel_l2(alt_logits, want_logits), "f32sum_agree": alt_next == want_next})
        tok = want_next
    _log(rows)
    gpu = np.median([r["rel_l2"] for r in rows])
    alt = np.median([r["f32sum_rel_l2"] for r in rows])
    assert gpu <= 3.0 * alt + 1e-3, (gpu, alt)
    a_gpu = np.mean([r["agree"] for r in rows])
    a_alt = np.mean([r["f32sum_agree"] for r in rows])
    assert a_gpu >= a_alt - 0.25, (a_gpu, a_alt)
